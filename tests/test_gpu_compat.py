"""GPU parity of the reference-named launchers outside the fused layer path:
X8 quantizer, chunk CSR tier, NVFP4 M=1 and M=8 tiers, INT8 shared expert,
NVFP4 -> INT8 arena build. Integer outputs (codes, scales, routing
inversion) are compared bit for bit with the oracle; FFN outputs within
max|y - r| / max|r| <= 1e-2 against fp64 recomputations of the same
arithmetic (dequantized weights, exact X8 activations).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import _oracle as orc
import qfm

pytestmark = pytest.mark.gpu

TOL = 1e-2
RNG = np.random.default_rng(11)
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


def _dev(a):
    return qfm.DevBuf.from_array(np.ascontiguousarray(a))


def _sync(lib):
    qfm.check(lib.qfm_device_sync(), "sync")
    qfm.status_check()


def _routing(T, pool=None, skew=0.0):
    """sel [T][K] distinct experts per row (from pool if given), wts [T][K] > 0 summing to 1."""
    cand = np.arange(E) if pool is None else np.asarray(pool)
    p = np.exp(skew * RNG.standard_normal(cand.size))
    p /= p.sum()
    sel = np.stack([RNG.choice(cand, K, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    w = RNG.random((T, K)).astype(np.float32) + 0.05
    return sel, (w / w.sum(1, keepdims=True)).astype(np.float32)


def _i8_expert_w(seed, layer, e):
    Qg = orc.fill("i8", seed, layer, orc.T_QG, e * I * H, I * H).reshape(I, H)
    Qu = orc.fill("i8", seed, layer, orc.T_QU, e * I * H, I * H).reshape(I, H)
    Qd = orc.fill("i8", seed, layer, orc.T_QD, e * H * I, H * I).reshape(H, I)
    sg = orc.fill("rowscale", seed, layer, orc.T_SG, e * I, I)
    su = orc.fill("rowscale", seed, layer, orc.T_SU, e * I, I)
    sd = orc.fill("rowscale", seed, layer, orc.T_SD, e * H, H)
    return Qg, sg, Qu, su, Qd, sd


def _f4_expert_w(seed, layer, e):
    Fg = orc.fill("fp4byte", seed, layer, orc.T_FG, e * I * H // 2, I * H // 2).reshape(I, H // 2)
    Fu = orc.fill("fp4byte", seed, layer, orc.T_FU, e * I * H // 2, I * H // 2).reshape(I, H // 2)
    Fd = orc.fill("fp4byte", seed, layer, orc.T_FD, e * H * I // 2, H * I // 2).reshape(H, I // 2)
    Sg = orc.fill("e4m3scale", seed, layer, orc.T_FSG, e * I * H // 16, I * H // 16).reshape(I, H // 16)
    Su = orc.fill("e4m3scale", seed, layer, orc.T_FSU, e * I * H // 16, I * H // 16).reshape(I, H // 16)
    Sd = orc.fill("e4m3scale", seed, layer, orc.T_FSD, e * H * I // 16, H * I // 16).reshape(H, I // 16)
    return Fg, Sg, Fu, Su, Fd, Sd


def _x8_rows(T):
    x = orc.bf16_to_f32(orc.fill("gauss_bf16", 5, 77, orc.T_X, 0, T * H)).reshape(T, H)
    q = np.empty((T, H), np.int8)
    s = np.empty((T, H // 32), np.float32)
    for t in range(T):
        q[t], s[t] = orc.x8_quant(x[t])
    xhat = q.astype(np.float64) * np.repeat(s.astype(np.float64), 32, axis=1)
    return q, s, xhat


# ------------------------------------------------------------------ X8
def test_x8_bit_exact(lib):
    _say("x8")
    v = (RNG.standard_normal(8192) * 3).astype(np.float32)
    v[64:96] = 0.0                                   # all-zero block -> scale 1
    v[128:160] = np.float32(1e-30) * RNG.standard_normal(32).astype(np.float32)
    v[300] = 1e30
    dv, dq, ds = _dev(v), qfm.DevBuf(v.size), qfm.DevBuf(v.size // 32 * 4)
    lib.qf8_i8_x8(dv.ptr, dq.ptr, ds.ptr, v.size, None)
    _sync(lib)
    q, s = orc.x8_quant(v)
    assert np.array_equal(dq.download(np.int8, v.size), q)
    assert np.array_equal(ds.download(np.float32, v.size // 32).view(np.uint32), s.view(np.uint32))


# ------------------------------------------------------------------ chunk CSR
@pytest.mark.parametrize("T,skew", [(1, 0.0), (7, 0.0), (300, 2.0), (8038, 3.0)])
def test_csr_build_bit_exact(lib, T, skew):
    _say("csr build", T, skew)
    sel, wt = _routing(T, skew=skew)
    ids, ptr, tok, kk, pw = orc.csr_build(sel, wt, E)
    P = T * K
    dsel, dwt = _dev(sel), _dev(wt)
    d_slot, d_ptr, d_tok, d_pw, d_cnt = (qfm.DevBuf(E * 4), qfm.DevBuf((E + 1) * 4), qfm.DevBuf(P * 4),
                                         qfm.DevBuf(P * 4), qfm.DevBuf(8))
    lib.qf8_i8_csr_build(dsel.ptr, dwt.ptr, T, d_slot.ptr, d_ptr.ptr, d_tok.ptr, d_pw.ptr, d_cnt.ptr, None)
    _sync(lib)
    cnt = d_cnt.download(np.int32, 2)
    n = len(ids)
    assert cnt[0] == n and cnt[1] == P
    assert np.array_equal(d_slot.download(np.int32, n), ids)
    assert np.array_equal(d_ptr.download(np.int32, n + 1), ptr)
    assert np.array_equal(d_tok.download(np.int32, P), tok)
    assert np.array_equal(d_pw.download(np.float32, P).view(np.uint32), pw.view(np.uint32))


@pytest.mark.parametrize("T", [1, 37, 129])
def test_experts_chunk(lib, T):
    """qf8_i8_experts_chunk: y[t] = sum_k w * expert_k(X8(x_t)), y overwritten."""
    seed, layer = 2, 4
    _say("experts chunk", T)
    pool = RNG.choice(E, 24, replace=False)
    sel, wt = _routing(T, pool=pool)
    q, s, xhat = _x8_rows(T)
    L = qfm.SynthLayer(qfm.QFM_FMT_INT8, seed, layer)
    P = T * K
    dsel, dwt, dq, ds = _dev(sel), _dev(wt), _dev(q), _dev(s)
    d_slot, d_ptr, d_tok, d_pw, d_cnt = (qfm.DevBuf(E * 4), qfm.DevBuf((E + 1) * 4), qfm.DevBuf(P * 4),
                                         qfm.DevBuf(P * 4), qfm.DevBuf(8))
    hid, part, y = qfm.DevBuf(P * I * 4), qfm.DevBuf(P * H * 4), _dev(np.full((T, H), 7.0, np.float32))
    lib.qf8_i8_csr_build(dsel.ptr, dwt.ptr, T, d_slot.ptr, d_ptr.ptr, d_tok.ptr, d_pw.ptr, d_cnt.ptr, None)
    lib.qf8_i8_experts_chunk(C.byref(L.s.arena), dq.ptr, ds.ptr, hid.ptr, None, None, d_slot.ptr, d_ptr.ptr,
                             d_tok.ptr, d_pw.ptr, d_cnt.ptr, min(P, E), P, dsel.ptr, part.ptr, T, y.ptr, None)
    _sync(lib)
    got = y.download(np.float32, (T, H))
    ref = np.zeros((T, H))
    cache = {}
    for t in range(T):
        for k in range(K):
            e = int(sel[t, k])
            if e not in cache:
                cache[e] = _i8_expert_w(seed, layer, e)
            _, ye = orc.i8_expert(xhat[t], *cache[e])
            ref[t] += float(wt[t, k]) * ye
    rel = max(_rel(got[t], ref[t]) for t in range(T))
    _say("  max rel err", rel)
    assert rel <= TOL
    L.destroy()


# ------------------------------------------------------------------ NVFP4 M=1
def test_nvfp4_m1_entry_points(lib):
    seed, layer = 3, 5
    _say("nvfp4 m1")
    L = qfm.SynthLayer(qfm.QFM_FMT_NVFP4, seed, layer)
    a = L.s.arena
    sel = RNG.choice(E, K, replace=False).astype(np.int32)
    slots = sel.copy()
    slots[3] = -1                                    # non-resident: zero hidden, no contribution
    wts = (RNG.random(K) + 0.1).astype(np.float32)
    x = orc.bf16_to_f32(orc.fill("gauss_bf16", seed, 99, orc.T_X, 0, H)).astype(np.float32)
    dx, dsel, dslot, dw = _dev(x), _dev(sel), _dev(slots), _dev(wts)
    hid, y1, y2 = qfm.DevBuf(K * I * 4), qfm.DevBuf(H * 4), qfm.DevBuf(H * 4)
    lib.qf5_nvfp4_moe_all(a.w_gate, a.s_gate, a.w_up, a.s_up, a.w_down, a.s_down, dx.ptr, hid.ptr, y1.ptr,
                          a.s2g_dev, a.s2u_dev, a.s2d_dev, dw.ptr, dsel.ptr, dslot.ptr, K, None)
    _sync(lib)
    h1 = hid.download(np.float32, (K, I))
    lib.qf5_nvfp4_gateup_all_launch(a.w_gate, a.s_gate, a.w_up, a.s_up, dx.ptr, hid.ptr, a.s2g_dev, a.s2u_dev,
                                    dsel.ptr, dslot.ptr, K, None)
    lib.qf5_nvfp4_downacc_all_launch(a.w_down, a.s_down, hid.ptr, dw.ptr, y2.ptr, a.s2d_dev, dsel.ptr, dslot.ptr,
                                     K, None)
    _sync(lib)
    g1, g2 = y1.download(np.float32, H), y2.download(np.float32, H)
    assert np.array_equal(g1, g2)
    assert not h1[3].any()
    ref = np.zeros(H)
    for k in range(K):
        if slots[k] < 0:
            continue
        Fg, Sg, Fu, Su, Fd, Sd = _f4_expert_w(seed, layer, int(sel[k]))
        hk, yk = orc.nvfp4_expert(x.astype(np.float64), Fg, Sg, 0.01, Fu, Su, 0.01, Fd, Sd, 0.01, H, I)
        assert _rel(h1[k], hk) <= TOL
        ref += float(wts[k]) * yk
    rel = _rel(g1, ref)
    _say("  max rel err", rel)
    assert rel <= TOL
    L.destroy()


# ------------------------------------------------------------------ NVFP4 M=8
@pytest.mark.parametrize("card,epc,il", [(0, 512, 0), (1, 128, 2)])
def test_m8_entry_points(lib, card, epc, il):
    seed, layer, M = 4, 6, 8
    _say("m8", card, epc, il)
    L = qfm.SynthLayer(qfm.QFM_FMT_NVFP4, seed, layer)
    a = L.s.arena
    sel, wt = _routing(M)
    if card:
        sel[:, 0] = 128 + np.arange(M) * 3           # every row has at least one expert in the range
    x = orc.bf16_to_f32(orc.fill("gauss_bf16", seed, 98, orc.T_X, 0, M * H)).reshape(M, H).astype(np.float32)
    P = M * K
    dsel, dwt, dx = _dev(sel), _dev(wt), _dev(x)
    d_slot, d_ptr, d_tok, d_pw, d_cnt = (qfm.DevBuf(P * 4), qfm.DevBuf((P + 1) * 4), qfm.DevBuf(P * 4),
                                         qfm.DevBuf(P * 4), qfm.DevBuf(8))
    lib.qf5_m8_build_csr(dsel.ptr, dwt.ptr, M, K, card, epc, il, d_slot.ptr, d_ptr.ptr, d_tok.ptr, d_pw.ptr,
                         d_cnt.ptr, None)
    _sync(lib)
    lo, hi = card * epc, card * epc + epc
    own = (sel >= lo) & (sel < hi)
    # oracle over the owned pairs only: stable order (expert, token, k)
    flat = sel.reshape(-1)
    keep = np.nonzero(own.reshape(-1))[0]
    order = keep[np.argsort(flat[keep], kind="stable")]
    exps = np.unique(flat[keep])
    cnt = d_cnt.download(np.int32, 2)
    assert cnt[0] == exps.size and cnt[1] == keep.size
    assert np.array_equal(d_slot.download(np.int32, exps.size), il * epc + (exps - lo))
    assert np.array_equal(d_ptr.download(np.int32, exps.size + 1),
                          np.concatenate([[0], np.cumsum([np.count_nonzero(flat[keep] == e) for e in exps])]))
    assert np.array_equal(d_tok.download(np.int32, keep.size), order // K)
    assert np.array_equal(d_pw.download(np.float32, keep.size), wt.reshape(-1)[order])
    # gate/up + down against the slots: for card > 0 the slot numbering is il*epc + local,
    # so point the weight bases at the first expert of the range shifted by the slot base.
    shift = lo - il * epc                            # expert = slot + shift
    GW, GS = I * H // 2, I * H // 16

    def base(p, per):
        return p + shift * per
    rt = qfm.Qf5M8Route(0, int(cnt[1]), M, P, d_cnt.ptr, d_slot.ptr, d_ptr.ptr, d_tok.ptr, d_pw.ptr)
    s2 = _dev(np.full(E + 1024, 0.01, np.float32))
    hid, yp = qfm.DevBuf(P * I * 4), _dev(np.zeros((M, H), np.float32))
    lib.qf5_m8_gateup(base(a.w_gate, GW), base(a.s_gate, GS), base(a.w_up, GW), base(a.s_up, GS), s2.ptr, s2.ptr,
                      dx.ptr, hid.ptr, C.byref(rt), None)
    lib.qf5_m8_downacc(base(a.w_down, GW), base(a.s_down, GS), s2.ptr, hid.ptr, yp.ptr, C.byref(rt), None)
    _sync(lib)
    got = yp.download(np.float32, (M, H))
    ref = np.zeros((M, H))
    for t in range(M):
        for k in range(K):
            if not own[t, k]:
                continue
            Fg, Sg, Fu, Su, Fd, Sd = _f4_expert_w(seed, layer, int(sel[t, k]))
            _, yk = orc.nvfp4_expert(x[t].astype(np.float64), Fg, Sg, 0.01, Fu, Su, 0.01, Fd, Sd, 0.01, H, I)
            ref[t] += float(wt[t, k]) * yk
    rows = [t for t in range(M) if own[t].any()]
    rel = max(_rel(got[t], ref[t]) for t in rows)
    _say("  max rel err", rel)
    assert rel <= TOL
    for t in range(M):
        if not own[t].any():
            assert not got[t].any()
    L.destroy()


# ------------------------------------------------------------------ shared expert
@pytest.mark.parametrize("T", [1, 5, 37])
def test_shexp_rows(lib, T):
    seed, layer = 6, 8
    _say("shexp", T)
    L = qfm.SynthLayer(qfm.QFM_FMT_INT8, seed, layer)
    lay = L.s.layer
    q, s, xhat = _x8_rows(T)
    gq = RNG.integers(-127, 128, (1, H), dtype=np.int8)
    gs = np.array([0.0004], np.float32)
    dgq, dgs = _dev(gq), _dev(gs)
    gi = qfm.Qf8I8Mat(dgq.ptr, dgs.ptr, 1, H)
    y0 = RNG.standard_normal((T, H)).astype(np.float32)
    dq, ds, y = _dev(q), _dev(s), _dev(y0)
    eg, eu, g1, ed = qfm.DevBuf(T * I * 4), qfm.DevBuf(T * I * 4), qfm.DevBuf(T * 4), qfm.DevBuf(T * H * 4)
    if T == 1:
        lib.qf8_i8_shexp_m1(C.byref(lay.sh_gate), C.byref(lay.sh_up), C.byref(gi), C.byref(lay.sh_down), dq.ptr,
                            ds.ptr, eg.ptr, eu.ptr, g1.ptr, ed.ptr, None, None, y.ptr, None)
    else:
        qfm.check(lib.qf8_i8_shexp_rows(C.byref(lay.sh_gate), C.byref(lay.sh_up), C.byref(gi), C.byref(lay.sh_down),
                                        dq.ptr, ds.ptr, eg.ptr, eu.ptr, g1.ptr, ed.ptr, None, None, y.ptr, T, None),
                  "shexp rows")
    _sync(lib)
    W = _i8_expert_w(seed, layer, E)                 # the shared expert is generator expert E
    got_y = y.download(np.float32, (T, H))
    got_g1 = g1.download(np.float32, T)
    got_ed = ed.download(np.float32, (T, H))
    for t in range(T):
        h, d = orc.i8_expert(xhat[t], *W)
        gl = float(gs[0]) * float(gq[0].astype(np.float64) @ xhat[t])
        assert abs(got_g1[t] - gl) <= 1e-4 * (abs(gl) + 1e-3)
        assert _rel(got_ed[t], d) <= TOL
        ref = y0[t].astype(np.float64) + d / (1 + np.exp(-gl))
        assert _rel(got_y[t] - y0[t], ref - y0[t]) <= TOL
    L.destroy()


# ------------------------------------------------------------------ NVFP4 -> INT8 build
def test_i8_build_bit_exact(lib):
    seed, layer = 7, 9
    _say("i8 build")
    L = qfm.SynthLayer(qfm.QFM_FMT_NVFP4, seed, layer)
    a = L.s.arena
    s2 = [(0.01 * (1 + np.arange(E) / 512 * (j + 1))).astype(np.float32) for j in range(3)]
    ds2 = [_dev(v) for v in s2]
    bufs = [qfm.DevBuf(E * I * H) for _ in range(3)] + [qfm.DevBuf(E * I * 4), qfm.DevBuf(E * I * 4),
                                                        qfm.DevBuf(E * H * 4)]
    c = qfm.Qf4ExpCache.from_buffer_copy(a)
    c.s2g_dev, c.s2u_dev, c.s2d_dev = ds2[0].ptr, ds2[1].ptr, ds2[2].ptr
    c.i8_gate, c.i8_up, c.i8_down = bufs[0].ptr, bufs[1].ptr, bufs[2].ptr
    c.i8s_gate, c.i8s_up, c.i8s_down = bufs[3].ptr, bufs[4].ptr, bufs[5].ptr
    assert lib.qf8_i8_build(C.byref(c), None) == 0
    _sync(lib)
    for e in (0, 17, 511):
        Fg, Sg, Fu, Su, Fd, Sd = _f4_expert_w(seed, layer, e)
        for F, S, j, rows, Kd in ((Fg, Sg, 0, I, H), (Fu, Su, 1, I, H), (Fd, Sd, 2, H, I)):
            qr, sr = orc.nvfp4_to_i8(F, S, float(s2[j][e]), rows, Kd)
            assert np.array_equal(bufs[j].download(np.int8, (rows, Kd), offset=e * I * H), qr), (e, j)
            assert np.array_equal(bufs[3 + j].download(np.float32, rows, offset=e * rows * 4).view(np.uint32),
                                  sr.view(np.uint32)), (e, j)
    # slot form: NVFP4 slot 17 -> INT8 slot 3 with expert 17's s2 equals the full build's slot 17
    assert lib.qf8_i8_build_slot(C.byref(c), 17, 3, 17, None) == 0
    _sync(lib)
    for j, rows in ((0, I), (1, I), (2, H)):
        assert np.array_equal(bufs[j].download(np.int8, I * H, offset=3 * I * H),
                              bufs[j].download(np.int8, I * H, offset=17 * I * H))
        assert np.array_equal(bufs[3 + j].download(np.float32, rows, offset=3 * rows * 4),
                              bufs[3 + j].download(np.float32, rows, offset=17 * rows * 4))
    L.destroy()


def test_m8_reduce4(lib):
    """qf5_m8_reduce4: bit-exact against the oracle's left-to-right fp32 sum, on
    the 16-byte path (aligned, n % 4 == 0 and ragged), the element path
    (pointers 4 bytes off alignment), in place (y_out == y0) and n == 0."""
    rng = np.random.default_rng(17)
    for n, off, inplace in ((8 * H, 0, False), (8 * H + 3, 0, False), (1001, 1, False), (7, 3, False),
                            (4 * H, 0, True), (5, 0, True)):
        _say("m8_reduce4", n, off, inplace)
        ys = [(rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 3, n)).astype(np.float32) for _ in range(4)]
        if n >= 4:                                   # the order-sensitive case in the first lanes
            ys[0][:2], ys[1][:2], ys[2][:2], ys[3][:2] = (2.0 ** 24, 1.0), (1.0, 1.0), (1.0, 1.0), (1.0, 2.0 ** 24)
        bufs = [_dev(np.concatenate([np.zeros(off, np.float32), v])) for v in ys]
        ptrs = [b.ptr + 4 * off for b in bufs]
        out = bufs[0] if inplace else qfm.DevBuf(4 * (n + off))
        optr = ptrs[0] if inplace else out.ptr + 4 * off
        lib.qf5_m8_reduce4(optr, *ptrs, n, None)
        _sync(lib)
        got = out.download(np.float32, n + off)[off:]
        ref = orc.m8_reduce4(*ys)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        if n >= 4:
            assert got[0] == 2.0 ** 24 and got[1] == 2.0 ** 24 + 4
    lib.qf5_m8_reduce4(None, None, None, None, None, 0, None)   # nothing to do, no error
    _sync(lib)
