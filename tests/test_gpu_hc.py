"""GPU: the dense INT8 x X8 GEMV, the FFN-side hyper-connection pre-mixer and
the stream inject against the oracle (ocho/amd_server/qf8_dense_i8.hip:78-175,
:360-375; qf8_hc.hip:99-103).

Bars: X8 codes/scales and the stream inject bit-exact (integer rule / one
fma on the same fp32 inputs); every fp32 stage within 2e-5 of max|ref|
relative, evaluated by the fp64 oracle on the GPU's own inputs to that stage;
the whole mixer (X8 rounding between stages) within 1e-2."""
import ctypes as C

import numpy as np
import pytest

import _oracle as orc
import qfm

pytestmark = pytest.mark.gpu

STAGE = 2e-5


def _say(*a):
    print(*a, flush=True)


def _rel(y, r):
    return float(np.abs(np.asarray(y, np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


@pytest.fixture(scope="module")
def lib():
    L = qfm.load()
    qfm.init(2560, 640, 512, 10, 1, 1)
    assert qfm.device_info()["arch"].startswith("gfx950")
    return L


class _Mat:
    """A device INT8 matrix with random codes and row scales."""

    def __init__(self, rng, rows, K, scale=0.01):
        self.q = rng.integers(-127, 128, (rows, K), dtype=np.int8)
        self.s = rng.uniform(0.5, 1.5, rows).astype(np.float32) * np.float32(scale)
        self.dq, self.ds = qfm.DevBuf.from_array(self.q), qfm.DevBuf.from_array(self.s)
        self.m = qfm.Qf8I8Mat(self.dq.ptr, self.ds.ptr, rows, K)


def _x8_rows(rng, T, K):
    x = rng.standard_normal((T, K)).astype(np.float32)
    qs = [orc.x8_quant(x[t]) for t in range(T)]
    return np.stack([q for q, _ in qs]), np.stack([s for _, s in qs])


@pytest.mark.parametrize("K", [320, 512, 640, 2048, 2560, 6144, 8192, 10240])
def test_gemv_multi_and_rows(lib, K):
    _say("gemv K", K)
    rng = np.random.default_rng(K)
    mats = [_Mat(rng, 100, K), _Mat(rng, 37, K), _Mat(rng, 1, K)]
    s = qfm.Stream()
    for T in (1, 5, 19):
        xq, xs = _x8_rows(rng, T, K)
        dxq, dxs = qfm.DevBuf.from_array(xq), qfm.DevBuf.from_array(xs)
        ys = [qfm.DevBuf(T * m.q.shape[0] * 4) for m in mats]
        mm = qfm.Qf8I8Multi()
        mm.n = 3
        for i, (m, y) in enumerate(zip(mats, ys)):
            mm.m[i] = C.pointer(m.m)
            mm.y[i] = y.ptr
            mm.act[i] = i
        if T == 1:
            assert lib.qf8_i8_gemv_multi_ex(C.byref(mm), dxq.ptr, dxs.ptr, s.h) == 0
        else:
            assert lib.qf8_i8_gemv_rows(C.byref(mm), dxq.ptr, dxs.ptr, T, s.h) == 0
        s.sync()
        for i, (m, y) in enumerate(zip(mats, ys)):
            got = y.download(np.float32, (T, m.q.shape[0]))
            for t in range(T):
                ref = orc.i8_gemv(m.q, m.s, xq[t], xs[t], i)
                assert _rel(got[t], ref) <= STAGE, (K, T, i, t)
    s.destroy()


def test_stream_inject_bit_exact(lib):
    rng = np.random.default_rng(5)
    H = 2560
    R = rng.standard_normal(4 * H).astype(np.float32)
    y = rng.standard_normal(H).astype(np.float32)
    inj = rng.uniform(0, 2, 4).astype(np.float32)
    dR, dy, di = qfm.DevBuf.from_array(R), qfm.DevBuf.from_array(y), qfm.DevBuf.from_array(inj)
    s = qfm.Stream()
    assert lib.qf8_stream_inject_ex(dR.ptr, dy.ptr, di.ptr, s.h) == 0
    s.sync()
    assert np.array_equal(dR.download(np.float32, (4 * H,)).view(np.uint32), orc.stream_inject(R, y, inj).view(np.uint32))
    s.destroy()


def _check_mixer(g, R1, R0, wn, mats, y_prev, inj_prev, fused, with_inject, H):
    """Every stage of T pre-mixer rows against the oracle on the GPU's own
    inputs to that stage; returns the worst end-to-end error of mixed."""
    down, inject, up = mats
    T = R0.shape[0]
    worst_e2e = 0.0
    for t in range(T):
        # fused inject: one fma per element, bit-exact
        Rt = orc.stream_inject(R0[t], y_prev[t], inj_prev[t]) if fused else R0[t]
        assert np.array_equal(R1[t].view(np.uint32), Rt.view(np.uint32))
        # norm on the GPU's residual, X8 of the GPU's normed
        nref = np.concatenate([orc.hc_norm(Rt[c * H:(c + 1) * H], wn[c * H:(c + 1) * H]) for c in range(4)])
        assert _rel(g["normed"][t], nref) <= STAGE
        q, sc = orc.x8_quant(g["normed"][t])
        assert np.array_equal(g["n8q"][t], q) and np.array_equal(g["n8s"][t].view(np.uint32), sc.view(np.uint32))
        # down / inject on the GPU's X8(normed)
        assert _rel(g["hc_d"][t], orc.i8_gemv(down.q, down.s, q, sc, 1)) <= STAGE
        if with_inject:
            assert _rel(g["inj"][t][:4], orc.i8_gemv(inject.q, inject.s, q, sc, 2)) <= STAGE
        dq, ds = orc.x8_quant(g["hc_d"][t])
        assert np.array_equal(g["d8q"][t], dq) and np.array_equal(g["d8s"][t].view(np.uint32), ds.view(np.uint32))
        assert _rel(g["hcy"][t], orc.i8_gemv(up.q, up.s, dq, ds, 0)) <= STAGE
        assert _rel(g["mixed"][t], orc.hc_combine(g["hcy"][t], g["normed"][t], H)) <= STAGE
        xq, xs = orc.x8_quant(g["mixed"][t])
        assert np.array_equal(g["xq"][t], xq) and np.array_equal(g["xs"][t].view(np.uint32), xs.view(np.uint32))
        # the whole mixer from the residual alone (the oracle's own X8 roundings between stages)
        n32 = nref.astype(np.float32)
        q2, s2 = orc.x8_quant(n32)
        h32 = orc.i8_gemv(down.q, down.s, q2, s2, 1).astype(np.float32)
        dq2, ds2 = orc.x8_quant(h32)
        hy = orc.i8_gemv(up.q, up.s, dq2, ds2, 0).astype(np.float32)
        e2e = _rel(g["mixed"][t], orc.hc_combine(hy, n32, H))
        worst_e2e = max(worst_e2e, e2e)
    return worst_e2e


@pytest.mark.parametrize("H,T,fused,with_inject", [(2560, 1, False, True), (2560, 1, True, True), (2048, 1, True, False),
                                                   (2560, 3, True, True), (2048, 4, False, True)])
def test_hc_premixer(lib, H, T, fused, with_inject):
    _say("hc premixer H", H, "T", T, "fused inject", fused, "inject", with_inject)
    qfm.init(H, H // 4, 512, 10, 1, 1)
    rng = np.random.default_rng(H + T)
    RS, L = 4 * H, 320
    down, inject, up = _Mat(rng, L, RS, 0.004), _Mat(rng, 4, RS, 0.004), _Mat(rng, RS, L, 0.02)
    R0 = rng.standard_normal((T, RS)).astype(np.float32)
    wn = (rng.uniform(-0.2, 0.2, RS).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    y_prev = rng.standard_normal((T, H)).astype(np.float32)
    inj_prev = rng.uniform(0, 2, (T, 4)).astype(np.float32)
    dR = qfm.DevBuf.from_array(R0)
    dwn = qfm.DevBuf.from_array(wn)
    dyp, dip = qfm.DevBuf.from_array(y_prev), qfm.DevBuf.from_array(inj_prev)
    out = {nm: qfm.DevBuf(T * n) for nm, n in (("normed", RS * 4), ("hc_d", L * 4), ("mixed", H * 4), ("inj", 16),
                                                 ("n8q", RS), ("n8s", RS // 32 * 4), ("d8q", L), ("d8s", L // 32 * 4),
                                                 ("hcy", RS * 4), ("xq", H), ("xs", H // 32 * 4))}
    s = qfm.Stream()
    args = [out["normed"].ptr, out["hc_d"].ptr, out["mixed"].ptr, out["inj"].ptr if with_inject else None, dR.ptr,
            dwn.ptr, C.byref(down.m), C.byref(inject.m) if with_inject else None, C.byref(up.m), out["n8q"].ptr,
            out["n8s"].ptr, out["d8q"].ptr, out["d8s"].ptr, out["hcy"].ptr, dyp.ptr if fused else None,
            dip.ptr if fused else None, out["xq"].ptr, out["xs"].ptr]
    rc = lib.qf8_i8_hc_m1_ex(*args, s.h) if T == 1 else lib.qf8_i8_hc_rows(*args, T, s.h)
    assert rc == 0, lib.qfm_last_error().decode()
    s.sync()
    g = {nm: b.download(dt, (T, b.nbytes // T // np.dtype(dt).itemsize)) for (nm, b), dt in
         zip(out.items(), (np.float32, np.float32, np.float32, np.float32, np.int8, np.float32, np.int8, np.float32,
                           np.float32, np.int8, np.float32))}
    R1 = dR.download(np.float32, (T, RS))
    worst_e2e = _check_mixer(g, R1, R0, wn, (down, inject, up), y_prev, inj_prev, fused, with_inject, H)
    _say("  end-to-end mixed rel err", worst_e2e)
    assert worst_e2e <= 1e-2
    s.destroy()
    qfm.init(2560, 640, 512, 10, 1, 1)


def test_hc_rejects_bad_shapes(lib):
    rng = np.random.default_rng(0)
    down, up = _Mat(rng, 320, 4 * 2560), _Mat(rng, 4 * 2560, 320)
    bad = _Mat(rng, 320, 4 * 2048)
    b = qfm.DevBuf(1 << 20)
    p = b.ptr
    common = [p, p, p, None, p, p]
    assert lib.qf8_i8_hc_m1_ex(*common, C.byref(bad.m), None, C.byref(up.m), p, p, p, p, p, None, None, p, p,
                               None) == -2
    assert lib.qf8_i8_hc_m1_ex(*common, C.byref(down.m), None, C.byref(up.m), p, p, p, p, p, p, None, p, p,
                               None) == -1                      # y_prev without inj_prev
    lib.qfm_last_error()


def _hc_bufs(T, H):
    RS, L = 4 * H, 320
    return {nm: qfm.DevBuf(T * n) for nm, n in (("normed", RS * 4), ("hc_d", L * 4), ("mixed", H * 4), ("inj", 16),
                                                ("n8q", RS), ("n8s", RS // 32 * 4), ("d8q", L), ("d8s", L // 32 * 4),
                                                ("hcy", RS * 4), ("xq", H), ("xs", H // 32 * 4), ("xb", H * 2))}


def _hc_call(lib, b, dR, dwn, mats, dyp, dip, with_inject, T, st):
    down, inject, up = mats
    args = [b["normed"].ptr, b["hc_d"].ptr, b["mixed"].ptr, b["inj"].ptr if with_inject else None, dR.ptr, dwn.ptr,
            C.byref(down.m), C.byref(inject.m) if with_inject else None, C.byref(up.m), b["n8q"].ptr, b["n8s"].ptr,
            b["d8q"].ptr, b["d8s"].ptr, b["hcy"].ptr, dyp.ptr if dyp else None, dip.ptr if dip else None,
            b["xq"].ptr, b["xs"].ptr, b["xb"].ptr, T, st.h]
    rc = lib.qfm_hc_premix(*args)
    assert rc == 0, lib.qfm_last_error().decode()


def _hc_bytes(b, T):
    return {nm: buf.download(np.uint8, (T, buf.nbytes // T)) for nm, buf in b.items()}


_HC_TYPES = {"normed": np.float32, "hc_d": np.float32, "mixed": np.float32, "inj": np.float32, "n8q": np.int8,
             "n8s": np.float32, "d8q": np.int8, "d8s": np.float32, "hcy": np.float32, "xq": np.int8, "xs": np.float32,
             "xb": np.uint16}


def _hc_typed(b, T):
    return {nm: buf.download(_HC_TYPES[nm], (T, buf.nbytes // T // np.dtype(_HC_TYPES[nm]).itemsize))
            for nm, buf in b.items()}


@pytest.mark.parametrize("H,with_inject,fused", [(2048, True, True), (2560, True, True), (2048, False, True),
                                                 (2560, True, False), (2048, False, False)])
def test_hc_one_launch_consecutive_and_graph(lib, H, with_inject, fused):
    """One row runs as one launch (slice blocks publish partial dots and normed
    as tagged words, up blocks wait for them); T rows run as two launches.
    Over consecutive one-row calls (the hand-off tag advancing) every stage
    matches the oracle, and normed, its X8 codes and the updated residual are
    the two-launch form's bits (the same norm partition); graph replays with
    eager calls between them give the eager bits; no bounded wait runs out."""
    _say("hc one launch: H", H, "inject", with_inject, "fused inject", fused)
    qfm.init(H, H // 4, 512, 10, 1, 1)
    rng = np.random.default_rng(7 * H + with_inject + 2 * fused)
    RS, L = 4 * H, 320
    mats = (_Mat(rng, L, RS, 0.004), _Mat(rng, 4, RS, 0.004), _Mat(rng, RS, L, 0.02))
    wn = (rng.uniform(-0.2, 0.2, RS).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    dwn = qfm.DevBuf.from_array(wn)
    st = qfm.Stream()
    before = C.c_uint32(0)
    assert lib.qfm_hc_wait_timeouts(C.byref(before)) == 0, lib.qfm_last_error().decode()
    one, two = _hc_bufs(1, H), _hc_bufs(2, H)
    for k in range(3):
        R0 = rng.standard_normal(RS).astype(np.float32)
        yp = rng.standard_normal(H).astype(np.float32)
        ip = rng.uniform(0, 2, 4).astype(np.float32)
        dyp = qfm.DevBuf.from_array(yp) if fused else None
        dip = qfm.DevBuf.from_array(ip) if fused else None
        dyp2 = qfm.DevBuf.from_array(np.stack([yp, yp])) if fused else None
        dip2 = qfm.DevBuf.from_array(np.stack([ip, ip])) if fused else None
        dR1, dR2 = qfm.DevBuf.from_array(R0), qfm.DevBuf.from_array(np.stack([R0, R0]))
        _hc_call(lib, one, dR1, dwn, mats, dyp, dip, with_inject, 1, st)
        _hc_call(lib, two, dR2, dwn, mats, dyp2, dip2, with_inject, 2, st)
        st.sync()
        a, b = _hc_typed(one, 1), _hc_typed(two, 2)
        r1, r2 = dR1.download(np.float32, (1, RS)), dR2.download(np.float32, (2, RS))
        e2e = _check_mixer(a, r1, R0[None], wn, mats, yp[None], ip[None], fused, with_inject, H)
        _say("  call", k, "end-to-end mixed rel err", e2e)
        assert e2e <= 1e-2
        for nm in ("normed", "n8q", "n8s"):
            assert np.array_equal(a[nm][0].view(np.uint8), b[nm][0].view(np.uint8)), (k, nm)
        assert np.array_equal(r1[0].view(np.uint32), r2[0].view(np.uint32)), k
        # the down / inject values differ from the two-launch form's by the summation order only
        for nm in ("hc_d",) + (("inj",) if with_inject else ()):
            assert _rel(a[nm][0][:4] if nm == "inj" else a[nm][0], (b[nm][0][:4] if nm == "inj" else b[nm][0])
                        .astype(np.float64)) <= STAGE, (k, nm)
    # graph: two one-row calls captured, replayed three times with eager calls between
    dRg = qfm.DevBuf.from_array(R0)
    g_out = [_hc_bufs(1, H), _hc_bufs(1, H)]
    qfm.check(lib.qfm_graph_capture_begin(st.h), "capture")
    for bo in g_out:
        _hc_call(lib, bo, dRg, dwn, mats, None, None, with_inject, 1, st)
    g = lib.qfm_graph_capture_end(st.h)
    assert g, lib.qfm_last_error().decode()
    dRe = qfm.DevBuf.from_array(R0)
    eager = _hc_bufs(1, H)
    _hc_call(lib, eager, dRe, dwn, mats, None, None, with_inject, 1, st)
    st.sync()
    want = _hc_bytes(eager, 1)
    for rep in range(3):
        for bo in g_out:
            for buf in bo.values():
                buf.zero()
        qfm.check(lib.qfm_graph_launch(g, st.h), "launch")
        st.sync()
        for bo in g_out:
            got = _hc_bytes(bo, 1)
            for nm in got:
                if nm == "inj" and not with_inject:
                    continue
                assert np.array_equal(got[nm], want[nm]), (rep, nm)
        _hc_call(lib, eager, dRe, dwn, mats, None, None, with_inject, 1, st)
        st.sync()
        again = _hc_bytes(eager, 1)
        assert all(np.array_equal(again[nm], want[nm]) for nm in want if nm != "inj" or with_inject), rep
    assert lib.qfm_graph_destroy(g) == 0
    after = C.c_uint32(0)
    assert lib.qfm_hc_wait_timeouts(C.byref(after)) == 0
    assert after.value == before.value, (before.value, after.value)
    st.destroy()
    qfm.init(2560, 640, 512, 10, 1, 1)
