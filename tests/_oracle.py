"""ctypes binding of the CPU oracle (oracle/_build/libqfm_oracle.so).

Test infrastructure: the checker the HIP path is compared against. Builds
the oracle with make on first use when the shared object is absent.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "_build", "libqfm_oracle.so")

T_QG, T_QU, T_QD, T_SG, T_SU, T_SD = 1, 2, 3, 4, 5, 6
T_ROUTER, T_X, T_SHGATE, T_BIAS = 7, 8, 9, 10
T_FG, T_FU, T_FD, T_FSG, T_FSU, T_FSD = 11, 12, 13, 14, 15, 16

vp = C.c_void_p
u32, u64 = C.c_uint32, C.c_uint64


class LayerCfg(C.Structure):
    _fields_ = [("H", C.c_int), ("I", C.c_int), ("E", C.c_int), ("K", C.c_int),
                ("fmt", C.c_int), ("gated", C.c_int), ("renorm", C.c_int), ("use_bias", C.c_int),
                ("seed", u32), ("layer", u32), ("x_layer", u32), ("x_row0", C.c_int)]


class HostLayer(C.Structure):
    _fields_ = [("router", vp), ("qg", vp), ("qu", vp), ("qd", vp),
                ("sg", vp), ("su", vp), ("sd", vp), ("shgate", vp)]


_SIGS = {
    "orc_philox4x32_10": (None, [vp, vp, vp]),
    "orc_word": (u32, [u32, u32, u32, u64]),
    "orc_gen_i8": (C.c_int8, [u32, u32, u32, u64]),
    "orc_gen_rowscale": (C.c_float, [u32, u32, u32, u64]),
    "orc_gen_gauss": (C.c_float, [u32, u32, u32, u64]),
    "orc_gen_fp4byte": (C.c_uint8, [u32, u32, u32, u64]),
    "orc_gen_e4m3scale": (C.c_uint8, [u32, u32, u32, u64]),
    "orc_fill_i8": (None, [u32, u32, u32, u64, u64, vp]),
    "orc_fill_rowscale": (None, [u32, u32, u32, u64, u64, vp]),
    "orc_fill_gauss": (None, [u32, u32, u32, u64, u64, C.c_float, vp]),
    "orc_fill_gauss_bf16": (None, [u32, u32, u32, u64, u64, vp]),
    "orc_fill_fp4byte": (None, [u32, u32, u32, u64, u64, vp]),
    "orc_fill_e4m3scale": (None, [u32, u32, u32, u64, u64, vp]),
    "orc_e2m1": (C.c_float, [u32]),
    "orc_e4m3": (C.c_float, [u32]),
    "orc_e4m3_encode": (C.c_uint8, [C.c_float]),
    "orc_bf16_rne": (C.c_uint16, [C.c_float]),
    "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
    "orc_router_logits": (None, [vp, vp, vp, C.c_int, C.c_int, C.c_int, vp]),
    "orc_topk": (None, [vp, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, vp]),
    "orc_i8_expert": (None, [vp, vp, vp, vp, vp, vp, vp, C.c_int, C.c_int, vp, vp]),
    "orc_nvfp4_expert": (None, [vp, vp, vp, C.c_float, vp, vp, C.c_float, vp, vp, C.c_float,
                                C.c_int, C.c_int, vp, vp]),
    "orc_nvfp4_dequant": (None, [vp, vp, C.c_float, C.c_int, C.c_int, vp]),
    "orc_x8_quant": (None, [vp, C.c_int, vp, vp]),
    "orc_nvfp4_to_i8": (None, [vp, vp, C.c_float, C.c_int, C.c_int, vp, vp]),
    "orc_i8_quant_bf16": (None, [vp, C.c_int, C.c_int, vp, vp]),
    "orc_f8_decode": (C.c_float, [C.c_uint8]),
    "orc_f8_encode": (C.c_uint8, [C.c_float]),
    "orc_fp8_pack_expert": (None, [vp, vp, C.c_float, C.c_int, C.c_int, vp, vp]),
    "orc_i8_gemv": (None, [vp, vp, C.c_int, C.c_int, vp, vp, C.c_int, vp]),
    "orc_hc_norm": (None, [vp, vp, C.c_int, vp]),
    "orc_hc_combine": (None, [vp, vp, C.c_int, vp]),
    "orc_stream_inject": (None, [vp, vp, vp, C.c_int]),
    "orc_shexp_bf16": (None, [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, vp, vp, vp, vp]),
    "orc_csr_build": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp, vp, vp, vp, vp]),
    "orc_m8_reduce4": (None, [vp, vp, vp, vp, vp, C.c_long]),
    "orc_moe_layer": (C.c_int, [C.POINTER(LayerCfg), C.c_int, vp, vp, vp, vp, vp, vp]),
    "orc_cpu_moe_layer_fast": (None, [C.POINTER(HostLayer), C.c_int, C.c_int, C.c_int, C.c_int,
                                      vp, C.c_int, vp, C.c_int]),
}

_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)
    lib = C.CDLL(ORACLE_SO)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def ptr(a):
    return a.ctypes.data if a is not None else None


# ---- numpy-facing helpers -------------------------------------------------
def philox(ctr, key):
    lib = load()
    c = np.array(ctr, dtype=np.uint32)
    k = np.array(key, dtype=np.uint32)
    o = np.zeros(4, dtype=np.uint32)
    lib.orc_philox4x32_10(ptr(c), ptr(k), ptr(o))
    return o


def fill(kind, seed, layer, tensor, n0, cnt, scale=1.0):
    lib = load()
    if kind == "i8":
        out = np.empty(cnt, np.int8); lib.orc_fill_i8(seed, layer, tensor, n0, cnt, ptr(out))
    elif kind == "rowscale":
        out = np.empty(cnt, np.float32); lib.orc_fill_rowscale(seed, layer, tensor, n0, cnt, ptr(out))
    elif kind == "gauss":
        out = np.empty(cnt, np.float32); lib.orc_fill_gauss(seed, layer, tensor, n0, cnt, scale, ptr(out))
    elif kind == "gauss_bf16":
        out = np.empty(cnt, np.uint16); lib.orc_fill_gauss_bf16(seed, layer, tensor, n0, cnt, ptr(out))
    elif kind == "fp4byte":
        out = np.empty(cnt, np.uint8); lib.orc_fill_fp4byte(seed, layer, tensor, n0, cnt, ptr(out))
    elif kind == "e4m3scale":
        out = np.empty(cnt, np.uint8); lib.orc_fill_e4m3scale(seed, layer, tensor, n0, cnt, ptr(out))
    else:
        raise ValueError(kind)
    return out


def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def router_logits(W, x_bf16, bias=None):
    lib = load()
    W = np.ascontiguousarray(W, np.float32)
    x = np.ascontiguousarray(x_bf16, np.uint16)
    E, H = W.shape
    M = x.shape[0]
    out = np.empty((M, E), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib.orc_router_logits(ptr(W), ptr(x), ptr(b), M, E, H, ptr(out))
    return out


def topk(logits, K, renorm=1):
    lib = load()
    lg = np.ascontiguousarray(logits, np.float32)
    M, E = lg.shape
    sel = np.empty((M, K), np.int32)
    w64 = np.empty((M, K), np.float64)
    w32 = np.empty((M, K), np.float32)
    lib.orc_topk(ptr(lg), M, E, K, renorm, ptr(sel), ptr(w64), ptr(w32))
    return sel, w64, w32


def i8_expert(x, Qg, sg, Qu, su, Qd, sd):
    lib = load()
    I, H = Qg.shape
    xd = np.ascontiguousarray(x, np.float64)
    h = np.empty(I, np.float64)
    y = np.empty(H, np.float64)
    args = [np.ascontiguousarray(a) for a in (Qg, sg, Qu, su, Qd, sd)]
    lib.orc_i8_expert(ptr(xd), *[ptr(a) for a in args], H, I, ptr(h), ptr(y))
    return h, y


def nvfp4_dequant(F, S, s2, rows, K):
    lib = load()
    out = np.empty((rows, K), np.float64)
    lib.orc_nvfp4_dequant(ptr(np.ascontiguousarray(F)), ptr(np.ascontiguousarray(S)), s2, rows, K, ptr(out))
    return out


def nvfp4_expert(x, Fg, Sg, s2g, Fu, Su, s2u, Fd, Sd, s2d, H, I):
    lib = load()
    xd = np.ascontiguousarray(x, np.float64)
    h = np.empty(I, np.float64)
    y = np.empty(H, np.float64)
    c = np.ascontiguousarray
    lib.orc_nvfp4_expert(ptr(xd), ptr(c(Fg)), ptr(c(Sg)), s2g, ptr(c(Fu)), ptr(c(Su)), s2u,
                         ptr(c(Fd)), ptr(c(Sd)), s2d, H, I, ptr(h), ptr(y))
    return h, y


def nvfp4_to_i8(F, S, s2, rows, K):
    lib = load()
    q = np.empty((rows, K), np.int8)
    sc = np.empty(rows, np.float32)
    lib.orc_nvfp4_to_i8(ptr(np.ascontiguousarray(F, np.uint8)), ptr(np.ascontiguousarray(S, np.uint8)), s2, rows, K,
                        ptr(q), ptr(sc))
    return q, sc


def i8_quant_bf16(W):
    """bf16 bits [rows][K] -> (int8 codes, fp32 row scales) by orc_i8_quant_bf16."""
    lib = load()
    W = np.ascontiguousarray(W, np.uint16)
    rows, K = W.shape
    q = np.empty((rows, K), np.int8)
    sc = np.empty(rows, np.float32)
    lib.orc_i8_quant_bf16(ptr(W), rows, K, ptr(q), ptr(sc))
    return q, sc


def f8_decode_table():
    """fp32 value of every FP8 lane-chunk code (orc_f8_decode), [256]."""
    lib = load()
    return np.array([lib.orc_f8_decode(b) for b in range(256)], np.float32)


def fp8_pack_expert(W, S, s2, rows, n_in):
    """NVFP4 matrix -> (E4M3 codes [rows][in], fp32 chunk scales [rows][64]) by orc_fp8_pack_expert."""
    lib = load()
    w8 = np.empty((rows, n_in), np.uint8)
    sc = np.empty((rows, 64), np.float32)
    lib.orc_fp8_pack_expert(ptr(np.ascontiguousarray(W, np.uint8)), ptr(np.ascontiguousarray(S, np.uint8)),
                            float(s2), rows, n_in, ptr(w8), ptr(sc))
    return w8, sc


def fp8_dequant(w8, sc):
    """fp64 weights of a lane-chunk matrix: decode(code) * chunk scale."""
    rows, n_in = w8.shape
    ch = n_in // 64
    v = f8_decode_table().astype(np.float64)[w8]
    return v * np.repeat(sc.astype(np.float64), ch, axis=1)


def i8_gemv(W, s, xq, xs, act=0):
    """INT8 [rows][K] x one X8 row -> fp64 [rows] (orc_i8_gemv)."""
    lib = load()
    W = np.ascontiguousarray(W, np.int8)
    rows, K = W.shape
    y = np.empty(rows, np.float64)
    lib.orc_i8_gemv(ptr(W), ptr(np.ascontiguousarray(s, np.float32)), rows, K, ptr(np.ascontiguousarray(xq, np.int8)),
                    ptr(np.ascontiguousarray(xs, np.float32)), act, ptr(y))
    return y


def hc_norm(R, w):
    lib = load()
    R = np.ascontiguousarray(R, np.float32)
    out = np.empty(R.shape[0], np.float64)
    lib.orc_hc_norm(ptr(R), ptr(np.ascontiguousarray(w, np.uint16)), R.shape[0], ptr(out))
    return out


def hc_combine(hcy, normed, H):
    lib = load()
    out = np.empty(H, np.float64)
    lib.orc_hc_combine(ptr(np.ascontiguousarray(hcy, np.float32)), ptr(np.ascontiguousarray(normed, np.float32)), H,
                       ptr(out))
    return out


def stream_inject(R, y, inj):
    lib = load()
    R = np.array(R, np.float32, copy=True)
    lib.orc_stream_inject(ptr(R), ptr(np.ascontiguousarray(y, np.float32)), ptr(np.ascontiguousarray(inj, np.float32)),
                          len(y))
    return R


def shexp_bf16(gate, up, down, gate_inp, x, y):
    """bf16 shared expert over the rows of x [M][H] (orc_shexp_bf16): (eg, eu, g1, ed, y + sigmoid(g1) * ed), fp64."""
    lib = load()
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    M, H = x.shape
    I = gate.shape[0]
    eg, eu, ed = np.empty((M, I)), np.empty((M, I)), np.empty((M, H))
    g1 = np.empty(M)
    yo = np.array(np.atleast_2d(y), np.float64, copy=True)
    lib.orc_shexp_bf16(ptr(np.ascontiguousarray(gate, np.uint16)), ptr(np.ascontiguousarray(up, np.uint16)),
                       ptr(np.ascontiguousarray(down, np.uint16)), ptr(np.ascontiguousarray(gate_inp, np.uint16)),
                       ptr(x), M, H, I, ptr(eg), ptr(eu), ptr(g1), ptr(ed), ptr(yo))
    return eg, eu, g1, ed, yo


def x8_quant(v):
    lib = load()
    v = np.ascontiguousarray(v, np.float32)
    q = np.empty(v.shape[0], np.int8)
    s = np.empty(v.shape[0] // 32, np.float32)
    lib.orc_x8_quant(ptr(v), v.shape[0], ptr(q), ptr(s))
    return q, s


def m8_reduce4(y0, y1, y2, y3):
    lib = load()
    ys = [np.ascontiguousarray(v, np.float32) for v in (y0, y1, y2, y3)]
    out = np.empty_like(ys[0])
    lib.orc_m8_reduce4(ptr(out), *[ptr(v) for v in ys], out.size)
    return out


def csr_build(sel, wt, E):
    lib = load()
    sel = np.ascontiguousarray(sel, np.int32)
    wt = np.ascontiguousarray(wt, np.float32)
    T, K = sel.shape
    exp_ids = np.empty(T * K, np.int32)
    exp_ptr = np.empty(T * K + 1, np.int32)
    pair_tok = np.empty(T * K, np.int32)
    pair_k = np.empty(T * K, np.int32)
    pair_wt = np.empty(T * K, np.float32)
    npairs = C.c_int()
    n = lib.orc_csr_build(ptr(sel), ptr(wt), T, K, E, ptr(exp_ids), ptr(exp_ptr), ptr(pair_tok),
                          ptr(pair_k), ptr(pair_wt), C.byref(npairs))
    if n < 0:
        raise ValueError("bad expert id")
    return exp_ids[:n], exp_ptr[:n + 1], pair_tok[:npairs.value], pair_k[:npairs.value], pair_wt[:npairs.value]


def moe_layer(H, I, E, K, M, seed, layer, x_layer, x_row0=0, fmt=0, gated=1, renorm=1, use_bias=0):
    lib = load()
    cfg = LayerCfg(H, I, E, K, fmt, gated, renorm, use_bias, seed, layer, x_layer, x_row0)
    x = np.empty((M, H), np.uint16)
    logits = np.empty((M, E), np.float32)
    sel = np.empty((M, K), np.int32)
    w64 = np.empty((M, K), np.float64)
    y64 = np.empty((M, H), np.float64)
    ybf = np.empty((M, H), np.uint16)
    rc = lib.orc_moe_layer(C.byref(cfg), M, ptr(x), ptr(logits), ptr(sel), ptr(w64), ptr(y64), ptr(ybf))
    assert rc == 0
    return dict(x=x, logits=logits, sel=sel, w=w64, y=y64, ybf=ybf)


def _i8_expert_arrays(seed, layer, e, H, I):
    """Generator arrays of INT8 expert e (the shared expert is e = E)."""
    Qg = fill("i8", seed, layer, T_QG, e * I * H, I * H).reshape(I, H)
    Qu = fill("i8", seed, layer, T_QU, e * I * H, I * H).reshape(I, H)
    Qd = fill("i8", seed, layer, T_QD, e * H * I, H * I).reshape(H, I)
    sg = fill("rowscale", seed, layer, T_SG, e * I, I)
    su = fill("rowscale", seed, layer, T_SU, e * I, I)
    sd = fill("rowscale", seed, layer, T_SD, e * H, H)
    return Qg, sg, Qu, su, Qd, sd


def _expert_fp64(seed, layer, e, H, I, fmt):
    """Expert e's gate, up, down weights as fp64 matrices (exact values:
    int8 * row scale, or e2m1 * e4m3 * s2 through orc_nvfp4_dequant)."""
    if fmt == 0:
        Qg, sg, Qu, su, Qd, sd = _i8_expert_arrays(seed, layer, e, H, I)
        return (Qg.astype(np.float64) * sg.astype(np.float64)[:, None],
                Qu.astype(np.float64) * su.astype(np.float64)[:, None],
                Qd.astype(np.float64) * sd.astype(np.float64)[:, None])
    IH = I * H
    Fg = fill("fp4byte", seed, layer, T_FG, e * IH // 2, IH // 2)
    Fu = fill("fp4byte", seed, layer, T_FU, e * IH // 2, IH // 2)
    Fd = fill("fp4byte", seed, layer, T_FD, e * IH // 2, IH // 2)
    Sg = fill("e4m3scale", seed, layer, T_FSG, e * IH // 16, IH // 16)
    Su = fill("e4m3scale", seed, layer, T_FSU, e * IH // 16, IH // 16)
    Sd = fill("e4m3scale", seed, layer, T_FSD, e * IH // 16, IH // 16)
    return (nvfp4_dequant(Fg, Sg, 0.01, I, H), nvfp4_dequant(Fu, Su, 0.01, I, H), nvfp4_dequant(Fd, Sd, 0.01, H, I))


def moe_layer_grouped(H, I, E, K, M, seed, layer, x_layer, x_row0=0, fmt=0, gated=1, renorm=1, use_bias=0, x=None,
                      router=None, expert_fn=None, shared=None, gate_vec=None, bias=None):
    """The whole layer (orc_moe_layer's definition) evaluated expert by expert:
    every distinct expert's weights are dequantized once (the oracle's own
    dequantization, exact in fp64) and applied to all of its tokens with fp64
    matrix products, so a T = 8038 prefill is checked in seconds. Routing comes
    from the oracle's router and top-K. x (bf16 bits [M][H]) overrides the
    generated input rows and router (fp32 [E][H]) the generated router weights;
    expert_fn(e) -> (Wg, Wu, Wd) fp64 overrides the routed experts, shared
    (Wg, Wu, Wd) the shared expert, gate_vec (fp32 [H]) its gate vector and
    bias (fp32 [E], with use_bias) the generated router bias.
    Same arithmetic as orc_moe_layer up to the order of fp64 summation (pinned
    against it in tests/test_oracle_path.py)."""
    if x is None:
        x = fill("gauss_bf16", seed, x_layer, T_X, x_row0 * H, M * H).reshape(M, H)
    W = fill("gauss", seed, layer, T_ROUTER, 0, E * H, 0.02).reshape(E, H) if router is None else router
    b = (fill("gauss", seed, layer, T_BIAS, 0, E, 1.5) if bias is None else bias) if use_bias else None
    logits = router_logits(W, x, b)
    sel, w64, _ = topk(logits, K, renorm)
    X = bf16_to_f32(x).astype(np.float64)
    y = np.zeros((M, H), np.float64)

    def expert_out(Wg, Wu, Wd, Xe):
        g = Xe @ Wg.T
        u = Xe @ Wu.T
        with np.errstate(over="ignore"):         # silu(g) -> -0 as exp(-g) -> inf for very negative g
            return (g / (1.0 + np.exp(-g)) * u) @ Wd.T

    for e in np.unique(sel):
        rows, ks = np.nonzero(sel == e)
        Wg, Wu, Wd = _expert_fp64(seed, layer, int(e), H, I, fmt) if expert_fn is None else expert_fn(int(e))
        y[rows] += w64[rows, ks][:, None] * expert_out(Wg, Wu, Wd, X[rows])
    # shared expert: generator INT8 expert index E unless given
    Wg, Wu, Wd = _expert_fp64(seed, layer, E, H, I, 0) if shared is None else shared
    ys = expert_out(Wg, Wu, Wd, X)
    if gated:
        g = (fill("gauss", seed, layer, T_SHGATE, 0, H, 0.02) if gate_vec is None else gate_vec).astype(np.float64)
        with np.errstate(over="ignore"):          # sigma -> 0 as exp(-v) -> inf
            ys *= (1.0 / (1.0 + np.exp(-(X @ g))))[:, None]
    y += ys
    return dict(x=x, logits=logits, sel=sel, w=w64, y=y)
