"""GPU parity on the edge cases of the decode formats and the selection:

* X8 quantization on exact ties (v = (k + 1/2) s): round half to even, bit-exact;
* prefill tokens whose x row is zero: every expert is a candidate (the
  candidate-overflow fallback), ties go to the lowest expert index, and the
  workspace counter reports those tokens;
* fork rows (M <= 8) whose experts coincide, all rows on the same ten experts
  or a mix of shared and private ones (each distinct expert's pair range
  staged past its first two rows);
* prefill selection on constructed near-ties: router rows whose bf16 roundings
  coincide, so the MFMA logits cannot order them and only the exact
  recomputation does;
* every E4M3 block-scale byte 0x00..0xFF (bytes >= 0x80 are large unsigned
  scales, 0x7F is +inf, as the reference decodes them) through every NVFP4
  decode path: the fused fork-row kernels, the prefill grouped GEMMs and the
  reference-named M=1 / M=8 tiers, against the oracle's dequantization of the
  same codes and scale bytes.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import _oracle as orc
import qfm

pytestmark = pytest.mark.gpu

TOL = 1e-2
H, I, E, K = 2048, 512, 512, 10


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    L = qfm.load()
    qfm.init(H, I, E, K, 1, 1)
    assert qfm.device_info()["arch"].startswith("gfx950")
    return L


def _rel(y, r):
    return float(np.abs(y - r).max() / np.abs(r).max())


def _sync(lib):
    qfm.check(lib.qfm_device_sync(), "sync")
    qfm.status_check()


def _forward(lib, lay, x_bits, st):
    """qfm_moe_forward on bf16 rows x_bits [M][H]; returns y (fp32 of the bf16
    output), sel, wts and the prefill counters (None for M <= 8)."""
    M = x_bits.shape[0]
    dx, dy = qfm.DevBuf.from_array(x_bits), qfm.DevBuf(M * H * 2)
    wsb = lib.qfm_workspace_bytes(M)
    ws = qfm.DevBuf(wsb)
    qfm.check(lib.qfm_moe_forward(C.byref(lay), dx.ptr, M, dy.ptr, ws.ptr, wsb, st.h), "forward")
    st.sync()
    view = qfm.QfmWsView()
    lib.qfm_workspace_view(ws.ptr, M, C.byref(view))
    out = dict(y=orc.bf16_to_f32(dy.download(np.uint16, (M, H))), sel=qfm.d2h(view.sel, np.int32, (M, K)),
               wts=qfm.d2h(view.wts, np.float32, (M, K)))
    out["counters"] = qfm.d2h(view.counters, np.int32, 3) if view.counters else None
    return out


# ------------------------------------------------------------------ X8 ties
def test_x8_ties_bit_exact(lib):
    """qf8_i8_x8 rounds exact ties half to even like the reference's rintf
    (qf8_moe_i8.hip:66): absmax 127 gives the scale 1.0 exactly."""
    _say("x8 ties")
    ties = np.array([0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, 126.5, -126.5, 5.5, 6.5, -7.5], np.float32)
    v = np.zeros(128, np.float32)
    for blk, sgn in ((0, 1), (1, -1), (2, 1), (3, -1)):
        v[32 * blk] = 127.0 * sgn
        v[32 * blk + 1:32 * blk + 1 + ties.size] = sgn * ties
    dv, dq, ds = qfm.DevBuf.from_array(v), qfm.DevBuf(v.size), qfm.DevBuf(v.size // 32 * 4)
    qfm.check(lib.qf8_i8_x8_ex(dv.ptr, dq.ptr, ds.ptr, v.size, None), "x8")
    _sync(lib)
    q, s = orc.x8_quant(v)
    gq = dq.download(np.int8, v.size)
    assert np.array_equal(gq, q)
    assert np.array_equal(ds.download(np.float32, v.size // 32).view(np.uint32), s.view(np.uint32))
    assert np.array_equal(gq[1:1 + ties.size], np.rint(ties).astype(np.int8))


# ------------------------------------------------------------------ prefill: zero rows
@pytest.mark.parametrize("bias", [False, True])
def test_prefill_zero_rows_fallback(lib, bias):
    """Zero x rows: without a router bias every approximate logit is 0, all 512
    experts become candidates (the overflow fallback), the exact logits are all
    0 and the selection is experts 0..9 (ties to the lower index) with equal
    weights; the counter reports exactly those rows. With a bias the logits are
    the bias values and the selection is their top 10."""
    T, seed, layer, xl = 40, 2, 31, 77
    zero = [0, 5, 17, 39]
    _say("prefill zero rows, bias", bias)
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    L = qfm.SynthLayer(qfm.QFM_FMT_INT8, seed, layer, with_bias=bias, stream=st)
    x = orc.fill("gauss_bf16", seed, xl, orc.T_X, 0, T * H).reshape(T, H)
    x[zero] = 0
    g = _forward(lib, L.s.layer, x, st)
    r = orc.moe_layer_grouped(H, I, E, K, T, seed, layer, xl, use_bias=int(bias), x=x)
    assert np.array_equal(g["sel"], r["sel"])
    assert np.allclose(g["wts"], r["w"], rtol=2e-6, atol=1e-7)
    if not bias:
        assert np.array_equal(g["sel"][zero], np.tile(np.arange(K), (len(zero), 1)))
        assert np.allclose(g["wts"][zero], 0.1, rtol=1e-6)
        assert g["counters"][0] == len(zero), g["counters"]
    else:
        assert g["counters"][0] == 0, g["counters"]
    assert not g["y"][zero].any() and not r["y"][zero].any()     # zero rows: every expert outputs 0
    rel = max(_rel(g["y"][t], r["y"][t]) for t in range(T) if t not in zero)
    _say("  max rel err", rel, "fallback rows", int(g["counters"][0]))
    assert rel <= TOL
    L.destroy()
    st.destroy()


# ------------------------------------------------------------------ prefill: tile boundaries
@pytest.mark.parametrize("T,fmt", [(128, 0), (129, 0), (256, 1), (383, 0)])
def test_prefill_tile_boundaries(lib, T, fmt):
    """A router bias of +64 on experts 100..109 (and -64 elsewhere) sends every
    token to exactly those ten experts: eleven groups (with the shared one) of
    T rows each, i.e. exactly full 128-row tiles (T = 128, 256), one spare row
    (129), or 127 rows over (383), and 502 experts with no rows at all. Routing
    bit-exact and every output row against the grouped fp64 oracle given the
    same bias."""
    seed, layer, xl = 4, 23, 91
    _say("prefill tile boundaries T", T, "fmt", fmt)
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    L = qfm.SynthLayer(fmt, seed, layer, with_bias=True, stream=st)
    st.sync()                      # the generator writes the layer on st: finish before overwriting the bias
    bias = np.full(E, -64.0, np.float32)
    bias[100:110] = 64.0 + np.arange(10, dtype=np.float32) * 0.25
    qfm.check(lib.qfm_memcpy_h2d(L.s.layer.router_bias, bias.ctypes.data, bias.nbytes), "bias")
    x = orc.fill("gauss_bf16", seed, xl, orc.T_X, 0, T * H).reshape(T, H)
    g = _forward(lib, L.s.layer, x, st)
    r = orc.moe_layer_grouped(H, I, E, K, T, seed, layer, xl, use_bias=1, x=x, fmt=fmt, bias=bias)
    assert set(np.unique(g["sel"])) == set(range(100, 110))
    assert np.array_equal(g["sel"], r["sel"])
    assert np.allclose(g["wts"], r["w"], rtol=2e-6, atol=1e-7)
    rel = max(_rel(g["y"][t], r["y"][t]) for t in range(T))
    _say("  max rel err", rel, "counters", g["counters"])
    assert rel <= TOL
    L.destroy()
    st.destroy()


# ------------------------------------------------------------------ fork rows sharing experts
@pytest.mark.parametrize("M,fmt,boost", [(2, 0, 64.0), (8, 0, 64.0), (8, 1, 64.0), (8, 0, 1.5), (5, 1, 1.5)])
def test_fork_rows_sharing_experts(lib, M, fmt, boost):
    """Fork rows (M <= 8) whose experts coincide: a router bias of +boost on
    experts 100..109 sends every row to exactly those ten (boost 64: each
    distinct expert carries all M rows, so the gate/up blocks stage rows past
    the first two of their pair range) or makes them likely without forcing
    them (boost 1.5 against logits of spread ~0.9: a mix of shared and
    private experts). Routing bit-exact,
    every row's y against the grouped fp64 oracle with the same bias."""
    seed, layer, xl = 6, 27, 93
    _say("fork rows sharing experts M", M, "fmt", fmt, "boost", boost)
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    L = qfm.SynthLayer(fmt, seed, layer, with_bias=True, stream=st)
    st.sync()
    forced = boost >= 32
    bias = np.full(E, -64.0, np.float32) if forced else np.zeros(E, np.float32)
    bias[100:110] = boost + np.arange(10, dtype=np.float32) * (0.25 if forced else 0.0)
    qfm.check(lib.qfm_memcpy_h2d(L.s.layer.router_bias, bias.ctypes.data, bias.nbytes), "bias")
    x = orc.fill("gauss_bf16", seed, xl, orc.T_X, 0, M * H).reshape(M, H)
    g = _forward(lib, L.s.layer, x, st)
    r = orc.moe_layer_grouped(H, I, E, K, M, seed, layer, xl, use_bias=1, x=x, fmt=fmt, bias=bias)
    assert np.array_equal(g["sel"], r["sel"])
    if forced:
        assert (np.sort(g["sel"], axis=1) == np.arange(100, 110)).all()
    shared = len(np.unique(g["sel"]))
    assert np.allclose(g["wts"], r["w"], rtol=2e-6, atol=1e-7)
    rel = max(_rel(g["y"][t], r["y"][t]) for t in range(M))
    _say("  distinct experts", shared, "of", M * K, "max rel err", rel)
    assert rel <= TOL
    L.destroy()
    st.destroy()


# ------------------------------------------------------------------ prefill: near ties
def test_prefill_near_ties_exact_order(lib):
    """Router rows built so that token 0's 9th..12th experts have identical bf16
    roundings (their MFMA logits are equal) while their exact logits differ by a
    few ulps, plus one exact duplicate (a true tie, lower index wins). The
    prefill selection must still equal the oracle's exact top-K for every token."""
    T, seed, layer, xl = 33, 3, 12, 88
    _say("prefill near ties")
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    L = qfm.SynthLayer(qfm.QFM_FMT_INT8, seed, layer, with_bias=False, stream=st)
    W = orc.fill("gauss", seed, layer, orc.T_ROUTER, 0, E * H, 0.02).reshape(E, H).copy()
    x = orc.fill("gauss_bf16", seed, xl, orc.T_X, 0, T * H).reshape(T, H)
    lg = orc.router_logits(W, x[:1])[0]
    order = np.argsort(-lg.astype(np.float64), kind="stable")
    base = int(order[8])                              # token 0's 9th expert
    targets = [int(e) for e in order[20:24]]          # rows that become near copies of it
    xf = orc.bf16_to_f32(x[0]).astype(np.float64)
    k_big = int(np.argmax(np.abs(xf)))
    for j, e in enumerate(targets):
        W[e] = W[base]
        if j < 3:
            # nudge one weight by a few fp32 ulps: its bf16 rounding is unchanged
            w = np.float32(W[base, k_big])
            W[e, k_big] = np.nextafter(w, np.float32(np.inf) if (j % 2) == (xf[k_big] > 0) else np.float32(-np.inf))
            for _ in range(j):
                W[e, k_big] = np.nextafter(W[e, k_big], np.float32(np.inf) if (j % 2) == (xf[k_big] > 0) else np.float32(-np.inf))
    bf = lambda a: (a.view(np.uint32) + 0x7FFF + ((a.view(np.uint32) >> 16) & 1)) >> 16
    for e in targets:
        assert np.array_equal(bf(W[e]), bf(W[base])), "bf16 roundings coincide"
    dW = qfm.DevBuf.from_array(W)
    lay = qfm.QfmLayer.from_buffer_copy(L.s.layer)
    lay.router = dW.ptr
    g = _forward(lib, lay, x, st)
    r = orc.moe_layer_grouped(H, I, E, K, T, seed, layer, xl, x=x, router=W)
    lg0 = orc.router_logits(W, x[:1])[0]
    _say("  token 0 logits of the tied rows", [float(lg0[e]) for e in [base] + targets], "sel", g["sel"][0].tolist())
    assert np.array_equal(g["sel"], r["sel"])
    assert np.allclose(g["wts"], r["w"], rtol=2e-6, atol=1e-7)
    assert _rel(g["y"][0], r["y"][0]) <= TOL
    L.destroy()
    st.destroy()


# ------------------------------------------------------------------ E4M3 bytes
ALL_BYTES = np.arange(256)
S2 = 0.01


def _e4m3(b):
    return np.array([orc.load().orc_e4m3(int(v)) for v in np.atleast_1d(b)], np.float64)


class _F4Layer:
    """An NVFP4 layer without a shared expert whose e4m3 scale arrays the test
    overwrites; codes and routing stay those of the generator."""

    def __init__(self, lib, seed, layer, bias):
        self.lib, self.seed, self.layer = lib, seed, layer
        self.st = qfm.Stream()
        self.L = qfm.SynthLayer(qfm.QFM_FMT_NVFP4, seed, layer, with_bias=bias, stream=self.st)
        self.st.sync()             # generated on st; the scales are then overwritten from the host
        lay = qfm.QfmLayer.from_buffer_copy(self.L.s.layer)
        lay.sh_gate, lay.sh_up, lay.sh_down, lay.sh_gate_inp = qfm.Qf8I8Mat(), qfm.Qf8I8Mat(), qfm.Qf8I8Mat(), None
        self.lay = lay
        self.a = self.L.s.arena
        self.cache = {}

    def set_scales(self, gate_up_byte=None, down_rows=None):
        """gate/up: every block of every expert = gate_up_byte; down: row c of
        every expert = down_rows[c] for all its blocks."""
        n_gu = E * I * H // 16
        if gate_up_byte is not None:
            qfm.check(self.lib.qfm_memset(self.a.s_gate, int(gate_up_byte), n_gu), "memset")
            qfm.check(self.lib.qfm_memset(self.a.s_up, int(gate_up_byte), n_gu), "memset")
        if down_rows is not None:
            pat = np.repeat(np.asarray(down_rows, np.uint8)[:, None], I // 16, axis=1)
            big = np.ascontiguousarray(np.tile(pat.ravel(), E))
            qfm.check(self.lib.qfm_memcpy_h2d(self.a.s_down, big.ctypes.data, big.nbytes), "h2d")

    def unit(self, e):
        """Expert e's codes read back from the device, dequantized with unit
        block scales (byte 0x38 = 1.0): Wg, Wu, Wd (times s2) in fp64."""
        if e not in self.cache:
            ones_g = np.full((I, H // 16), 0x38, np.uint8)
            ones_d = np.full((H, I // 16), 0x38, np.uint8)
            GW = I * H // 2
            Fg = qfm.d2h(self.a.w_gate + e * GW, np.uint8, (I, H // 2))
            Fu = qfm.d2h(self.a.w_up + e * GW, np.uint8, (I, H // 2))
            Fd = qfm.d2h(self.a.w_down + e * GW, np.uint8, (H, I // 2))
            self.cache[e] = (orc.nvfp4_dequant(Fg, ones_g, S2, I, H), orc.nvfp4_dequant(Fu, ones_g, S2, I, H),
                             orc.nvfp4_dequant(Fd, ones_d, S2, H, I))
        return self.cache[e]

    def check_arrays(self, gate_up_byte, down_rows, experts):
        """The scale bytes the kernels read are the planted ones."""
        for e in list(experts)[:2]:
            sg = qfm.d2h(self.a.s_gate + e * (I * H // 16), np.uint8, I * H // 16)
            sd = qfm.d2h(self.a.s_down + e * (H * I // 16), np.uint8, (H, I // 16))
            assert (sg == gate_up_byte).all()
            assert np.array_equal(sd[:, 0], np.asarray(down_rows, np.uint8))

    def ref(self, x, sel, wts, sg_scale, sd_row_scale):
        """y[t] = sum_k w_k Wd_k (silu(s Wg_k x) * (s Wu_k x)) with the block
        scales applied as exact factors (the dequantized weight is
        e2m1 * e4m3 * s2, a product exact in fp64)."""
        X = orc.bf16_to_f32(x).astype(np.float64) if x.dtype == np.uint16 else x.astype(np.float64)
        y = np.zeros((X.shape[0], H))
        for t in range(X.shape[0]):
            for k in range(sel.shape[1]):
                Wg, Wu, Wd = self.unit(int(sel[t, k]))
                g = sg_scale * (Wg @ X[t])
                u = sg_scale * (Wu @ X[t])
                with np.errstate(over="ignore", invalid="ignore"):
                    h = g / (1.0 + np.exp(-g)) * u
                    y[t] += float(wts[t, k]) * (sd_row_scale * (Wd @ h))
        return y

    def destroy(self):
        self.L.destroy()
        self.st.destroy()


def _paths(lib, F, x_rows, x_pf, rng):
    """Run every NVFP4 decode path on the current scale bytes. Returns a list of
    (name, y, x, sel, wts)."""
    out = []
    g = _forward(lib, F.lay, x_rows, F.st)                       # fused fork-row kernels (M = 2)
    out.append(("fused M=2", g["y"], x_rows, g["sel"], g["wts"]))
    p = _forward(lib, F.lay, x_pf, F.st)                         # prefill grouped GEMMs (T = 9)
    out.append(("prefill T=9", p["y"], x_pf, p["sel"], p["wts"]))
    a = F.a
    x1 = orc.bf16_to_f32(x_rows[0]).astype(np.float32)
    sel = rng.choice(E, K, replace=False).astype(np.int32)
    wts = (rng.random(K) + 0.1).astype(np.float32)
    dx, dsel, dw = qfm.DevBuf.from_array(x1), qfm.DevBuf.from_array(sel), qfm.DevBuf.from_array(wts)
    hid, y1 = qfm.DevBuf(K * I * 4), qfm.DevBuf(H * 4)
    qfm.check(lib.qf5_nvfp4_moe_all_ex(a.w_gate, a.s_gate, a.w_up, a.s_up, a.w_down, a.s_down, dx.ptr, hid.ptr, y1.ptr,
                                       a.s2g_dev, a.s2u_dev, a.s2d_dev, dw.ptr, dsel.ptr, dsel.ptr, K, None), "moe_all")
    _sync(lib)
    out.append(("compat M=1", y1.download(np.float32, (1, H)), x1[None, :], sel[None, :], wts[None, :]))
    return out


@pytest.fixture(scope="module")
def f4(lib):
    qfm.init(H, I, E, K, 1, 1)
    F = _F4Layer(lib, 9, 21, bias=True)
    yield F
    F.destroy()


def test_e4m3_every_gate_up_byte(lib, f4):
    """Each of the 255 finite scale bytes (0x7F = +inf would make every output
    NaN) in turn as the gate and up block scale of every expert, down scales 1.0:
    the fused fork-row, prefill and reference-named M=1 paths against the
    oracle's dequantization. Bytes >= 0x80 are scales up to 2^24 * 1.875."""
    _say("e4m3 gate/up bytes")
    x_rows = orc.fill("gauss_bf16", 9, 501, orc.T_X, 0, 2 * H).reshape(2, H)
    x_pf = orc.fill("gauss_bf16", 9, 502, orc.T_X, 0, 9 * H).reshape(9, H)
    f4.set_scales(down_rows=np.full(H, 0x38, np.uint8))
    bytes_ = [b for b in ALL_BYTES if b != 0x7F]
    runs = {}                                        # path -> (x, sel, wts, [y per byte])
    for b in bytes_:
        f4.set_scales(gate_up_byte=b)
        _sync(lib)
        if b in (0x00, 0x80, 0xFF):
            f4.check_arrays(b, np.full(H, 0x38, np.uint8), [0])
        for name, y, x, sel, wts in _paths(lib, f4, x_rows, x_pf, np.random.default_rng(0)):
            if name not in runs:
                runs[name] = (x, sel, wts, [])
            else:                                    # routing does not depend on the expert weights
                assert np.array_equal(runs[name][1], sel), name
            runs[name][3].append(y)
    scales = _e4m3(np.array(bytes_))
    for name, (x, sel, wts, ys) in runs.items():
        Y = np.stack(ys)                                              # [byte][rows][H]
        R = np.zeros_like(Y, dtype=np.float64)
        X = orc.bf16_to_f32(x).astype(np.float64) if x.dtype == np.uint16 else x.astype(np.float64)
        for t in range(X.shape[0]):
            for k in range(sel.shape[1]):
                Wg, Wu, Wd = f4.unit(int(sel[t, k]))
                g = np.outer(scales, Wg @ X[t])                       # [byte][I]
                u = np.outer(scales, Wu @ X[t])
                with np.errstate(over="ignore", invalid="ignore"):
                    h = g / (1.0 + np.exp(-g)) * u
                R[:, t] += float(wts[t, k]) * (h @ Wd.T)
        worst = 0.0
        for i, b in enumerate(bytes_):
            if scales[i] == 0.0:
                assert not Y[i].any(), (name, b)
                continue
            rel = max(_rel(Y[i, t], R[i, t]) for t in range(X.shape[0]))
            worst = max(worst, rel)
            assert rel <= TOL, (name, hex(b), rel)
        _say("  ", name, "worst rel err over the 255 finite bytes", worst)


def test_e4m3_every_down_byte(lib, f4):
    """Down block scales: row c of every expert takes byte c % 256 (all 256
    bytes, eight rows each; gate/up scales 1.0). Rows with a 0x7F (+inf) scale
    must come out non-finite and leave the other rows finite; every other byte's
    rows are checked against the oracle relative to their own magnitude, and a
    zero scale gives exact zeros."""
    _say("e4m3 down bytes")
    rng = np.random.default_rng(4)
    x_rows = orc.fill("gauss_bf16", 9, 503, orc.T_X, 0, 2 * H).reshape(2, H)
    x_pf = orc.fill("gauss_bf16", 9, 504, orc.T_X, 0, 9 * H).reshape(9, H)
    rows = (np.arange(H) % 256).astype(np.uint8)
    f4.set_scales(gate_up_byte=0x38, down_rows=rows)
    _sync(lib)
    f4.check_arrays(0x38, rows, [0])
    srow = _e4m3(rows)
    finite = np.isfinite(srow)
    paths = _paths(lib, f4, x_rows, x_pf, rng)
    # the reference-named M=8 tier (atomic down into a pre-zeroed y), 8 rows
    a = f4.a
    M = 8
    x8 = orc.fill("gauss_bf16", 9, 505, orc.T_X, 0, M * H).reshape(M, H)
    xf = orc.bf16_to_f32(x8).astype(np.float32)
    sel = np.stack([rng.choice(E, K, replace=False) for _ in range(M)]).astype(np.int32)
    wt = (rng.random((M, K)) + 0.1).astype(np.float32)
    P = M * K
    dsel, dwt, dx = qfm.DevBuf.from_array(sel), qfm.DevBuf.from_array(wt), qfm.DevBuf.from_array(xf)
    d_slot, d_ptr, d_tok, d_pw, d_cnt = (qfm.DevBuf(P * 4), qfm.DevBuf((P + 1) * 4), qfm.DevBuf(P * 4),
                                         qfm.DevBuf(P * 4), qfm.DevBuf(8))
    qfm.check(lib.qf5_m8_build_csr_ex(dsel.ptr, dwt.ptr, M, K, 0, E, 0, d_slot.ptr, d_ptr.ptr, d_tok.ptr, d_pw.ptr,
                                      d_cnt.ptr, None), "csr")
    _sync(lib)
    cnt = d_cnt.download(np.int32, 2)
    rt = qfm.Qf5M8Route(0, int(cnt[1]), M, P, d_cnt.ptr, d_slot.ptr, d_ptr.ptr, d_tok.ptr, d_pw.ptr)
    hid, yp = qfm.DevBuf(P * I * 4), qfm.DevBuf.from_array(np.zeros((M, H), np.float32))
    qfm.check(lib.qf5_m8_gateup_ex(a.w_gate, a.s_gate, a.w_up, a.s_up, a.s2g_dev, a.s2u_dev, dx.ptr, hid.ptr,
                                   C.byref(rt), None), "m8 gateup")
    qfm.check(lib.qf5_m8_downacc_ex(a.w_down, a.s_down, a.s2d_dev, hid.ptr, yp.ptr, C.byref(rt), None), "m8 down")
    _sync(lib)
    paths.append(("compat M=8", yp.download(np.float32, (M, H)), xf, sel, wt))
    for name, y, x, sel_, wts_ in paths:
        r = f4.ref(x, sel_, wts_, 1.0, np.where(finite, srow, 0.0))
        assert np.isfinite(y[:, finite]).all(), name
        assert not np.isfinite(y[:, ~finite]).any(), name           # the 0x7F rows
        worst = 0.0
        for b in range(256):
            if b == 0x7F:
                continue
            cols = np.nonzero(rows == b)[0]
            ref_b, got_b = r[:, cols], y[:, cols]
            if srow[b] == 0.0:
                assert not got_b.any(), (name, b)
                continue
            rel = float(np.abs(got_b - ref_b).max() / np.abs(ref_b).max())
            worst = max(worst, rel)
            assert rel <= TOL, (name, hex(b), rel)
        _say("  ", name, "worst rel err over the 255 finite bytes", worst)


# ------------------------------------------------------------------ decode: zero rows
@pytest.mark.parametrize("M,fmt,bias", [(1, 0, False), (3, 0, False), (1, 1, True), (5, 1, False)])
def test_decode_zero_rows(lib, M, fmt, bias):
    """All-zero x rows through the fused decode paths (at M = 1 the INT8 gate/up
    kernel's own selection): without a bias every logit is 0, the selection is
    experts 0..9 (ties to the lower index) with weights 0.1; with a bias the
    logits are the bias and the selection its top 10. Every expert's output is
    0, so y is 0."""
    _say("decode zero rows M", M, "fmt", fmt, "bias", bias)
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    L = qfm.SynthLayer(fmt, 5, 61, with_bias=bias, stream=st)
    st.sync()
    x = np.zeros((M, H), np.uint16)
    g = _forward(lib, L.s.layer, x, st)
    r = orc.moe_layer_grouped(H, I, E, K, M, 5, 61, 0, use_bias=int(bias), x=x, fmt=fmt)
    assert np.array_equal(g["sel"], r["sel"])
    assert np.allclose(g["wts"], r["w"], rtol=2e-6, atol=1e-7)
    if not bias:
        assert np.array_equal(g["sel"], np.tile(np.arange(K), (M, 1)))
        assert np.allclose(g["wts"], 0.1, rtol=1e-6)
    assert not g["y"].any() and not r["y"].any()
    L.destroy()
    st.destroy()


# ------------------------------------------------------------------ dynamic range of x
@pytest.mark.parametrize("M,fmt,shift", [(1, 0, 24), (1, 0, -24), (4, 1, 24), (4, 0, -24), (40, 0, 24), (40, 1, -24)])
def test_input_dynamic_range(lib, M, fmt, shift):
    """x rows scaled by 2^shift (exact in bf16) through the fused decode and
    prefill paths: the activations as fp16 scaled per token or per 16 values,
    the hidden vectors' fp16 chunks and the prefill's scaled fp16 partials must
    follow the magnitude. At 2^24 the softmax is one-hot, at 2^-24 nearly
    uniform; the routing stays bit-exact and y within the usual bound."""
    _say("dynamic range M", M, "fmt", fmt, "shift", shift)
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    L = qfm.SynthLayer(fmt, 7, 71, with_bias=False, stream=st)
    st.sync()
    x0 = orc.fill("gauss_bf16", 7, 600 + M, orc.T_X, 0, M * H).reshape(M, H)
    xf = orc.bf16_to_f32(x0) * np.float32(2.0 ** shift)
    x = (xf.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(orc.bf16_to_f32(x), xf)                 # the scaling is exact
    g = _forward(lib, L.s.layer, x, st)
    r = orc.moe_layer_grouped(H, I, E, K, M, 7, 71, 0, x=x, fmt=fmt)
    assert np.array_equal(g["sel"], r["sel"])
    assert np.allclose(g["wts"], r["w"], rtol=2e-6, atol=1e-7)
    assert np.isfinite(g["y"]).all()
    rel = max(_rel(g["y"][t], r["y"][t]) for t in range(M))
    _say("  max rel err", rel)
    assert rel <= TOL
    L.destroy()
    st.destroy()
