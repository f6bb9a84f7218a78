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
