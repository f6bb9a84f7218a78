"""GPU: one GPU's shard of the tensor-parallel decode layout (every expert's
intermediate dimension split 8 ways: H 2048, I 512 / 8 = 64 per GPU; the
router and the shared expert's gate logit replicated). The M = 1 INT8 forward
at that shape against the fp64 oracle (logits and top-K bit-exact, y within
1e-2, bf16 and fp32 outputs); the paths built only for the full shapes reject
it with -2 and launch nothing."""
import ctypes as C

import numpy as np
import pytest

import _oracle as orc
import qfm

pytestmark = pytest.mark.gpu
H, I, E, K = 2048, 64, 512, 10
SEED, LAYER = 21, 9


def _say(*a):
    print("[shard]", *a, flush=True)


@pytest.fixture(scope="module")
def lib():
    L = qfm.load()
    qfm.init(H, I, E, K, 1, 1)
    yield L
    qfm.init(2048, 512, E, K, 1, 1)


@pytest.mark.parametrize("x_layer", [100, 101, 102])
def test_shard_m1_forward(lib, x_layer):
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    layer = qfm.SynthLayer(qfm.QFM_FMT_INT8, SEED, LAYER, stream=st)
    x = qfm.DevBuf(H * 2)
    qfm.check(lib.qfm_gen_input_rows(x.ptr, 1, SEED, x_layer, 0, st.h), "x")
    wsb = lib.qfm_workspace_bytes(1)
    ws, y, y32 = qfm.DevBuf(wsb), qfm.DevBuf(H * 2), qfm.DevBuf(H * 4)
    L = C.byref(layer.s.layer)
    qfm.check(lib.qfm_moe_forward(L, x.ptr, 1, y.ptr, ws.ptr, wsb, st.h), "forward")
    st.sync()
    view = qfm.QfmWsView()
    lib.qfm_workspace_view(ws.ptr, 1, C.byref(view))
    logits = qfm.d2h(view.logits, np.float32, (E + 1,))[:E]
    sel = qfm.d2h(view.sel, np.int32, (K,))
    ybf = y.download(np.uint16, (H,))
    qfm.check(lib.qfm_moe_forward_f32(L, x.ptr, 1, y32.ptr, ws.ptr, wsb, st.h), "forward f32")
    st.sync()
    yf = y32.download(np.float32, (H,))
    r = orc.moe_layer_grouped(H, I, E, K, 1, SEED, LAYER, x_layer)
    ref = orc.router_logits(orc.fill("gauss", SEED, LAYER, orc.T_ROUTER, 0, E * H, 0.02).reshape(E, H), r["x"])
    assert np.array_equal(logits.view(np.uint32), ref[0].view(np.uint32))
    assert np.array_equal(sel, r["sel"][0])
    yr = r["y"][0]
    eb = float(np.abs(orc.bf16_to_f32(ybf).astype(np.float64) - yr).max() / np.abs(yr).max())
    ef = float(np.abs(yf.astype(np.float64) - yr).max() / np.abs(yr).max())
    _say(f"x_layer {x_layer}: rel err bf16 y {eb:.2e}, fp32 y {ef:.2e}")
    assert eb <= 1e-2 and ef <= 1e-2
    layer.destroy()
    st.destroy()


def test_shard_rejects_unbuilt_paths(lib):
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    layer = qfm.SynthLayer(qfm.QFM_FMT_INT8, SEED, LAYER, stream=st)
    M = 3
    x = qfm.DevBuf(M * H * 2)
    qfm.check(lib.qfm_gen_input_rows(x.ptr, M, SEED, 100, 0, st.h), "x")
    wsb = lib.qfm_workspace_bytes(M)
    ws, y = qfm.DevBuf(wsb), qfm.DevBuf(M * H * 2)
    assert lib.qfm_moe_forward(C.byref(layer.s.layer), x.ptr, M, y.ptr, ws.ptr, wsb, st.h) == -2
    assert b"shape" in lib.qfm_last_error()
    assert lib.qf8_i8_shexp_rows(C.byref(layer.s.layer.sh_gate), C.byref(layer.s.layer.sh_up),
                                 C.byref(layer.s.layer.sh_gate), C.byref(layer.s.layer.sh_down), x.ptr, x.ptr,
                                 y.ptr, y.ptr, y.ptr, y.ptr, None, None, y.ptr, 1, st.h) == -2
    lib.qfm_last_error()
    st.sync()
    assert lib.qfm_status() == 0
    layer.destroy()
    st.destroy()
