"""GPU: the multi-layer forward (qfm_moe_forward_layers) and its graph-captured
replay, as bench.py times them.

A captured chain of layers is replayed several times, with the program's own
eager work and synchronizations between the replays, and every replay must
give the bits of the eager run of the same chain (the kernels write each
output once, in a fixed order, so eager and replayed results are identical).
The chain covers M = 1 (the single-row INT8 kernels), M = 8 (the fork-row
kernels, INT8 and NVFP4) and M = 4 NVFP4 (the selection in the router launch
and the combine in the down launch, whose tags advance on every replay), and
a prefill (T = 37: the counters cleared by a fill kernel, never by a memset
node).
"""
import ctypes as C
import sys

import numpy as np
import pytest

import _oracle as orc
import qfm

pytestmark = pytest.mark.gpu

H = 2048


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    L = qfm.load()
    qfm.init(H, 512, 512, 10, 1, 1)
    assert qfm.device_info()["arch"].startswith("gfx950")
    return L


@pytest.mark.parametrize("M,fmt,nl", [(1, 0, 4), (8, 0, 3), (8, 1, 3), (4, 1, 3), (37, 0, 2)])
def test_graph_replays_match_eager(lib, M, fmt, nl):
    _say("graph chain M", M, "fmt", fmt, "layers", nl)
    qfm.init(H, 512, 512, 10, 1, 1)
    st = qfm.Stream()
    layers = [qfm.SynthLayer(fmt, 0, 40 + l, with_bias=M > 8, stream=st) for l in range(nl)]
    arr = (qfm.QfmLayer * nl)(*[L.s.layer for L in layers])
    x = qfm.DevBuf(nl * M * H * 2)
    for l in range(nl):
        qfm.check(lib.qfm_gen_input_rows(x.ptr + l * M * H * 2, M, 0, 500 + l, 0, st.h), "x")
    y_eager, y_graph = qfm.DevBuf(nl * M * H * 2), qfm.DevBuf(nl * M * H * 2)
    wsb = lib.qfm_workspace_bytes(M)
    ws = qfm.DevBuf(wsb)

    def fwd(y):
        qfm.check(lib.qfm_moe_forward_layers(arr, nl, x.ptr, M * H, M, y.ptr, M * H, ws.ptr, wsb, st.h), "fwd")

    fwd(y_eager)
    st.sync()
    ref = y_eager.download(np.uint16, (nl, M, H))
    # the eager chain itself against the oracle on its last layer (the chain
    # passes each layer its own x rows and output rows)
    r = orc.moe_layer(H, 512, 512, 10, M, 0, 40 + nl - 1, 500 + nl - 1, fmt=fmt, use_bias=int(M > 8))
    got = orc.bf16_to_f32(ref[nl - 1])
    rel = float(np.abs(got - r["y"]).max() / np.abs(r["y"]).max())
    _say("  last layer max rel err", rel)
    assert rel <= 1e-2

    qfm.check(lib.qfm_graph_capture_begin(st.h), "capture")
    fwd(y_graph)
    g = lib.qfm_graph_capture_end(st.h)
    assert g, lib.qfm_last_error().decode()
    other = qfm.DevBuf(nl * M * H * 2)
    for rep in range(3):
        y_graph.zero()
        qfm.check(lib.qfm_graph_launch(g, st.h), "launch")
        st.sync()
        assert np.array_equal(y_graph.download(np.uint16, (nl, M, H)), ref), f"replay {rep}"
        # eager work on the same workspace between replays
        fwd(other)
        st.sync()
        assert np.array_equal(other.download(np.uint16, (nl, M, H)), ref), f"eager after replay {rep}"
    assert lib.qfm_graph_destroy(g) == 0
    for L in layers:
        L.destroy()
    st.destroy()
