"""qfm_moe_forward_noalloc (the fused forward on the library's built-in device
workspace, for callers that cannot allocate) against qfm_moe_forward with a
caller workspace: the same kernels, so the outputs must agree bit for bit, on
consecutive calls that shrink the input (the built-in array keeps the previous
call's contents)."""
import ctypes as C
import sys

import numpy as np
import pytest

import qfm

pytestmark = pytest.mark.gpu

H, I, E, K = 2048, 512, 512, 10


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _pair(lib, lay, M, seed, x_layer, st):
    dx, y_ref, y_na = qfm.DevBuf(M * H * 2), qfm.DevBuf(M * H * 2), qfm.DevBuf(M * H * 2)
    qfm.check(lib.qfm_gen_input_rows(dx.ptr, M, seed, x_layer, 0, st.h), "x")
    wsb = lib.qfm_workspace_bytes(M)
    ws = qfm.DevBuf(wsb)
    qfm.check(lib.qfm_moe_forward(C.byref(lay), dx.ptr, M, y_ref.ptr, ws.ptr, wsb, st.h), "forward")
    qfm.check(lib.qfm_moe_forward_noalloc(C.byref(lay), dx.ptr, M, y_na.ptr, st.h), "forward_noalloc")
    st.sync()
    qfm.status_check("noalloc")
    a, b = y_ref.download(np.uint16, (M, H)), y_na.download(np.uint16, (M, H))
    return a, b


@pytest.mark.parametrize("fmt", [qfm.QFM_FMT_INT8, qfm.QFM_FMT_NVFP4])
def test_noalloc_matches_workspace_forward(fmt):
    lib = qfm.load()
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    L = qfm.SynthLayer(fmt, 3, 40 + fmt, stream=st)
    for M, xl in ((8, 11), (3, 12), (1, 13)):      # each call smaller than the one before
        _say("noalloc fmt", fmt, "M", M)
        a, b = _pair(lib, L.s.layer, M, 3, xl, st)
        assert a.any()
        assert np.array_equal(a, b), (fmt, M)
    # beyond the built-in workspace: rejected, nothing launched
    assert lib.qfm_moe_forward_noalloc(C.byref(L.s.layer), None, 9, None, st.h) == -1
    assert b"1 <= M <= 8" in lib.qfm_last_error()
    L.destroy()
    st.destroy()


def test_noalloc_under_graph_capture():
    """The use the entry point exists for: captured into a graph (no
    allocation, no memset node), a chain of an M = 8 and an M = 1 forward on
    the built-in workspace replays three times, with eager calls between the
    replays, each bit-identical to the eager run."""
    lib = qfm.load()
    qfm.init(H, I, E, K, 1, 1)
    st = qfm.Stream()
    L8 = qfm.SynthLayer(qfm.QFM_FMT_INT8, 3, 50, stream=st)
    L1 = qfm.SynthLayer(qfm.QFM_FMT_NVFP4, 3, 51, stream=st)
    x8, x1 = qfm.DevBuf(8 * H * 2), qfm.DevBuf(H * 2)
    qfm.check(lib.qfm_gen_input_rows(x8.ptr, 8, 3, 21, 0, st.h), "x8")
    qfm.check(lib.qfm_gen_input_rows(x1.ptr, 1, 3, 22, 0, st.h), "x1")
    y8, y1 = qfm.DevBuf(8 * H * 2), qfm.DevBuf(H * 2)

    def chain():
        qfm.check(lib.qfm_moe_forward_noalloc(C.byref(L8.s.layer), x8.ptr, 8, y8.ptr, st.h), "noalloc M=8")
        qfm.check(lib.qfm_moe_forward_noalloc(C.byref(L1.s.layer), x1.ptr, 1, y1.ptr, st.h), "noalloc M=1")

    chain()
    st.sync()
    r8, r1 = y8.download(np.uint16, (8, H)), y1.download(np.uint16, (1, H))
    assert r8.any() and r1.any()
    qfm.check(lib.qfm_graph_capture_begin(st.h), "capture")
    chain()
    g = lib.qfm_graph_capture_end(st.h)
    assert g, lib.qfm_last_error().decode()
    for rep in range(3):
        _say("noalloc graph replay", rep)
        y8.zero()
        y1.zero()
        qfm.check(lib.qfm_graph_launch(g, st.h), "launch")
        st.sync()
        assert np.array_equal(y8.download(np.uint16, (8, H)), r8), rep
        assert np.array_equal(y1.download(np.uint16, (1, H)), r1), rep
        chain()                               # eager calls on the same built-in workspace
        st.sync()
    assert lib.qfm_graph_destroy(g) == 0
    L8.destroy()
    L1.destroy()
    st.destroy()
