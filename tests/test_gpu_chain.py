"""GPU: the FFN step the engine runs around the MoE, chained end to end
(ocho/amd_server/qf_hip4_stage.hip:1508-1644): the hyper-connection
pre-mixer emits the MoE input, the MoE layer writes y, the stream inject
writes it back into the residual. Each chain starts from the same residual
R0 on both sides and is compared with the oracle's own chain (fp64 stages,
the same X8 rules): the updated residual's change inj * y within 1e-2 of its
largest magnitude, the routing identical.

  fast chain       qfm_hc_premix (bf16(mixed) out) -> qfm_moe_forward_f32
                   (fp32 y) -> qf8_stream_inject, at one row (both shapes),
                   3 fork rows and 37 rows (the prefill path);
  reference chain  qf8_i8_hc_m1 (X8(mixed) out) -> INT8 router GEMV
                   (qf8_i8_gemv_multi) -> qf_rtr_topk10_launch ->
                   qf8_i8_gateup_m1 (quant_x = 0: the mixer's X8 row) ->
                   qf8_i8_down_m1 (seeds y) -> qf8_i8_shexp_m1 (adds the
                   gated shared expert) -> qf8_stream_inject, at the
                   reference's 2560/640 shape."""
import ctypes as C

import numpy as np
import pytest

import _oracle as orc
import qfm

pytestmark = pytest.mark.gpu
SEED, LAYER = 11, 4
TOL = 1e-2
HCL = 320


def _say(*a):
    print("[chain]", *a, flush=True)


def _rel(y, r):
    return float(np.abs(np.asarray(y, np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


class _Mat:
    """A device INT8 matrix with random codes and row scales."""

    def __init__(self, rng, rows, K, scale):
        self.q = rng.integers(-127, 128, (rows, K), dtype=np.int8)
        self.s = (rng.uniform(0.5, 1.5, rows) * scale).astype(np.float32)
        self.dq, self.ds = qfm.DevBuf.from_array(self.q), qfm.DevBuf.from_array(self.s)
        self.m = qfm.Qf8I8Mat(self.dq.ptr, self.ds.ptr, rows, K)


def _bf16_rne(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _mixer(rng, H):
    RS = 4 * H
    down, inject, up = _Mat(rng, HCL, RS, 0.004), _Mat(rng, 4, RS, 0.004), _Mat(rng, RS, HCL, 0.02)
    wn = (rng.uniform(-0.2, 0.2, RS).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return down, inject, up, wn


def _oracle_mixer(R, wn, down, inject, up, H):
    """One row of the pre-mixer in fp64 stages: (inj, mixed, X8(mixed))."""
    normed = np.concatenate([orc.hc_norm(R[c * H:(c + 1) * H], wn[c * H:(c + 1) * H]) for c in range(4)])
    q, sc = orc.x8_quant(normed.astype(np.float32))
    hc_d = orc.i8_gemv(down.q, down.s, q, sc, 1)
    inj = orc.i8_gemv(inject.q, inject.s, q, sc, 2)
    dq, ds = orc.x8_quant(hc_d.astype(np.float32))
    hcy = orc.i8_gemv(up.q, up.s, dq, ds, 0)
    mixed = orc.hc_combine(hcy.astype(np.float32), normed.astype(np.float32), H)
    xq, xs = orc.x8_quant(mixed.astype(np.float32))
    return inj, mixed, xq, xs


def _mixer_bufs(T, H):
    RS = 4 * H
    return {nm: qfm.DevBuf(T * n) for nm, n in (("normed", RS * 4), ("hc_d", HCL * 4), ("mixed", H * 4), ("inj", 16),
                                                  ("n8q", RS), ("n8s", RS // 32 * 4), ("d8q", HCL),
                                                  ("d8s", HCL // 32 * 4), ("hcy", RS * 4), ("xq", H),
                                                  ("xs", H // 32 * 4), ("xb", H * 2))}


def _mixer_args(b, dR, dwn, down, inject, up):
    return [b["normed"].ptr, b["hc_d"].ptr, b["mixed"].ptr, b["inj"].ptr, dR.ptr, dwn.ptr, C.byref(down.m),
            C.byref(inject.m), C.byref(up.m), b["n8q"].ptr, b["n8s"].ptr, b["d8q"].ptr, b["d8s"].ptr, b["hcy"].ptr,
            None, None, b["xq"].ptr, b["xs"].ptr]


@pytest.fixture(scope="module")
def lib():
    L = qfm.load()
    assert qfm.device_info()["arch"].startswith("gfx950")
    return L


@pytest.mark.parametrize("H,T", [(2048, 1), (2560, 1), (2048, 3), (2048, 37)])
def test_fast_chain(lib, H, T):
    I, E, K = H // 4, 512, 10
    _say("fast chain H", H, "rows", T)
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    layer = qfm.SynthLayer(qfm.QFM_FMT_INT8, SEED, LAYER, stream=st)
    rng = np.random.default_rng(H + T)
    RS = 4 * H
    down, inject, up, wn = _mixer(rng, H)
    R0 = rng.standard_normal((T, RS)).astype(np.float32)
    dR, dwn = qfm.DevBuf.from_array(R0), qfm.DevBuf.from_array(wn)
    b = _mixer_bufs(T, H)
    assert lib.qfm_hc_premix(*_mixer_args(b, dR, dwn, down, inject, up), b["xb"].ptr, T, st.h) == 0, \
        lib.qfm_last_error().decode()
    wsb = lib.qfm_workspace_bytes(T)
    ws, y = qfm.DevBuf(wsb), qfm.DevBuf(T * H * 4)
    assert lib.qfm_moe_forward_f32(C.byref(layer.s.layer), b["xb"].ptr, T, y.ptr, ws.ptr, wsb, st.h) == 0, \
        lib.qfm_last_error().decode()
    for t in range(T):
        assert lib.qf8_stream_inject_ex(dR.ptr + t * RS * 4, y.ptr + t * H * 4, b["inj"].ptr + t * 16, st.h) == 0
    st.sync()
    R1 = dR.download(np.float32, (T, RS))
    xb_gpu = b["xb"].download(np.uint16, (T, H))
    view = qfm.QfmWsView()
    lib.qfm_workspace_view(ws.ptr, T, C.byref(view))
    sel_gpu = qfm.d2h(view.sel, np.int32, (T, K))
    # the oracle's chain from R0
    injs, xs_ref = [], []
    for t in range(T):
        inj, mixed, _, _ = _oracle_mixer(R0[t], wn, down, inject, up, H)
        injs.append(inj)
        xs_ref.append(_bf16_rne(mixed))
    x_ref = np.stack(xs_ref)
    xv = lambda h: (h.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    bf_diff = _rel(xv(xb_gpu), xv(x_ref))
    r = orc.moe_layer_grouped(H, I, E, K, T, SEED, LAYER, 0, x=x_ref)
    assert np.array_equal(r["sel"], sel_gpu), "routing differs between the chains"
    worst = 0.0
    for t in range(T):
        d_ref = np.outer(injs[t], r["y"][t]).reshape(-1)
        worst = max(worst, _rel(R1[t].astype(np.float64) - R0[t], d_ref))
    _say(f"  bf16(mixed) vs the oracle's: {bf_diff:.1e} of max; worst rel err of R - R0: {worst:.2e}")
    assert worst <= TOL
    layer.destroy()
    st.destroy()


def test_reference_chain_x8(lib):
    """The engine's own M = 1 sequence of reference-named launchers, the
    mixer's X8 row handed to the router, the experts and the shared expert."""
    H, I, E, K = 2560, 640, 512, 10
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    layer = qfm.SynthLayer(qfm.QFM_FMT_INT8, SEED, LAYER, stream=st)
    arena = layer.s.arena
    rng = np.random.default_rng(7)
    RS = 4 * H
    down, inject, up, wn = _mixer(rng, H)
    router = _Mat(rng, E, H, 0.0008)
    shg, shu, shd = _Mat(rng, I, H, 0.002), _Mat(rng, I, H, 0.002), _Mat(rng, H, I, 0.004)
    shgi = _Mat(rng, 1, H, 0.002)
    R0 = rng.standard_normal(RS).astype(np.float32)
    dR, dwn = qfm.DevBuf.from_array(R0), qfm.DevBuf.from_array(wn)
    b = _mixer_bufs(1, H)
    logits, sel, wts = qfm.DevBuf(E * 4), qfm.DevBuf(16 * 4), qfm.DevBuf(16 * 4)
    hid, y = qfm.DevBuf(16 * I * 4), qfm.DevBuf(H * 4)
    h8q, h8s = qfm.DevBuf(16 * I), qfm.DevBuf(16 * I // 32 * 4)
    eg, eu, g1, ed = qfm.DevBuf(I * 4), qfm.DevBuf(I * 4), qfm.DevBuf(4), qfm.DevBuf(H * 4)
    e8q, e8s = qfm.DevBuf(I), qfm.DevBuf(I // 32 * 4)
    lib.qf8_i8_hc_m1(*_mixer_args(b, dR, dwn, down, inject, up), st.h)
    mm = qfm.Qf8I8Multi()
    mm.n = 1
    mm.m[0] = C.pointer(router.m)
    mm.y[0] = logits.ptr
    mm.act[0] = 0
    lib.qf8_i8_gemv_multi(C.byref(mm), b["xq"].ptr, b["xs"].ptr, st.h)
    lib.qf_rtr_topk10_launch(logits.ptr, sel.ptr, wts.ptr, st.h)
    lib.qf8_i8_gateup_m1(C.byref(arena), None, b["xq"].ptr, b["xs"].ptr, hid.ptr, sel.ptr, K, 0, st.h)
    lib.qf8_i8_down_m1(C.byref(arena), hid.ptr, h8q.ptr, h8s.ptr, wts.ptr, sel.ptr, y.ptr, K, st.h)
    lib.qf8_i8_shexp_m1(C.byref(shg.m), C.byref(shu.m), C.byref(shgi.m), C.byref(shd.m), b["xq"].ptr, b["xs"].ptr,
                        eg.ptr, eu.ptr, g1.ptr, ed.ptr, e8q.ptr, e8s.ptr, y.ptr, st.h)
    lib.qf8_stream_inject(dR.ptr, y.ptr, b["inj"].ptr, st.h)
    st.sync()
    assert lib.qfm_status() == 0, lib.qfm_last_error().decode()
    R1 = dR.download(np.float32, (RS,))
    xq_gpu = b["xq"].download(np.int8, (H,))
    sel_gpu = sel.download(np.int32, (16,))[:K]
    # oracle chain from R0 (X8 rows as in the reference)
    inj, _, xq, xs = _oracle_mixer(R0, wn, down, inject, up, H)
    x8_diff = int(np.abs(xq.astype(np.int32) - xq_gpu.astype(np.int32)).max())
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    lg = orc.i8_gemv(router.q, router.s, xq, xs, 0)
    order = np.lexsort((np.arange(E), -lg))[:K]                 # descending, ties to the lower index
    assert np.array_equal(order, sel_gpu), (order, sel_gpu)
    p = np.exp(lg[order] - lg[order[0]])
    w = p / p.sum()
    yv = np.zeros(H)
    for k, e in enumerate(order):
        Qg, sg, Qu, su, Qd, sd = orc._i8_expert_arrays(SEED, LAYER, int(e), H, I)
        g = (Qg.astype(np.float64) @ xd) * sg
        u = (Qu.astype(np.float64) @ xd) * su
        yv += w[k] * ((Qd.astype(np.float64) @ (g / (1 + np.exp(-g)) * u)) * sd)
    gs = orc.i8_gemv(shg.q, shg.s, xq, xs, 0)
    us = orc.i8_gemv(shu.q, shu.s, xq, xs, 0)
    gi = orc.i8_gemv(shgi.q, shgi.s, xq, xs, 0)[0]
    hs = gs / (1 + np.exp(-gs)) * us
    yv += (1 / (1 + np.exp(-gi))) * ((shd.q.astype(np.float64) @ hs) * shd.s)
    err = _rel(R1.astype(np.float64) - R0, np.outer(inj, yv).reshape(-1))
    _say(f"reference chain: X8(mixed) codes differ by at most {x8_diff}; rel err of R - R0: {err:.2e}")
    assert err <= TOL
    layer.destroy()
    st.destroy()
