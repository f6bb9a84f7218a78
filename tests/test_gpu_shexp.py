"""GPU: the bf16 shared expert of the NVFP4 stage (qf8_shexp / qf8_shexp_M,
ocho/amd_server/qf8_layer.hip:23-54) through the C ABI, against the fp64
oracle (orc_shexp_bf16) at both shapes: eg, eu, g1, ed and the gated add into
y, with y rows at a stride above H; argument rejection."""
import ctypes as C

import numpy as np
import pytest

import qfm
import _oracle as orc

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[shexp]", *a, flush=True)


def _bf16(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _rel(a, r):
    return float(np.max(np.abs(a - r)) / max(np.max(np.abs(r)), 1e-30))


@pytest.fixture(scope="module")
def lib():
    return qfm.load()


@pytest.mark.parametrize("shape", [(2048, 512), (2560, 640)])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_shexp_bf16_vs_oracle(lib, shape, M):
    H, I = shape
    _say("H", H, "I", I, "M", M)
    qfm.init(H, I, 512, 10, 1, 1)
    rng = np.random.default_rng(100 * M + H)
    gb, ub = _bf16(rng.standard_normal((I, H)) * 0.03), _bf16(rng.standard_normal((I, H)) * 0.03)
    db, ib = _bf16(rng.standard_normal((H, I)) * 0.03), _bf16(rng.standard_normal(H) * 0.05)
    x = rng.standard_normal((M, H)).astype(np.float32)
    ys = H + 64
    y0 = rng.standard_normal((M, ys)).astype(np.float32)
    d = {k: qfm.DevBuf.from_array(v) for k, v in (("g", gb), ("u", ub), ("d", db), ("i", ib), ("x", x), ("y", y0))}
    eg, eu, g1, ed = qfm.DevBuf(M * I * 4), qfm.DevBuf(M * I * 4), qfm.DevBuf(M * 4), qfm.DevBuf(M * H * 4)
    w = qfm.Qf8ShexpW(d["g"].ptr, d["u"].ptr, d["d"].ptr, d["i"].ptr)
    st = qfm.Stream()
    if M == 1:
        lib.qf8_shexp(C.byref(w), d["x"].ptr, eg.ptr, eu.ptr, g1.ptr, ed.ptr, d["y"].ptr, st.h)
        assert lib.qfm_status() == 0, lib.qfm_last_error()
        ys = H
        y0 = y0.reshape(-1)[:H].reshape(1, H)
    else:
        assert lib.qf8_shexp_M_ex(C.byref(w), d["x"].ptr, M, eg.ptr, eu.ptr, g1.ptr, ed.ptr, d["y"].ptr, I, ys,
                                  st.h) == 0, lib.qfm_last_error()
    st.sync()
    reg, reu, rg1, red, ry = orc.shexp_bf16(gb, ub, db, ib, x, y0[:, :H])
    got_y = d["y"].download(np.float32, (M, ys))
    errs = {"eg": _rel(eg.download(np.float32, (M, I)), reg), "eu": _rel(eu.download(np.float32, (M, I)), reu),
            "g1": _rel(g1.download(np.float32, (M,)), rg1), "ed": _rel(ed.download(np.float32, (M, H)), red),
            "y": _rel(got_y[:, :H], ry)}
    _say("  rel errs", {k: f"{v:.2e}" for k, v in errs.items()})
    assert max(errs.values()) <= 2e-5, errs
    if M > 1:   # the stride padding is untouched
        assert np.array_equal(got_y[:, H:], y0[:, H:])
    st.destroy()


def test_shexp_bf16_rejects(lib):
    qfm.init(2048, 512, 512, 10, 1, 1)
    buf = qfm.DevBuf(1 << 20)
    p = buf.ptr
    w = qfm.Qf8ShexpW(p, p, p, p)
    for M, ys in ((0, 2048), (9, 2048), (2, 2047)):
        assert lib.qf8_shexp_M_ex(C.byref(w), p, M, p, p, p, p, p, 512, ys, None) == -1
        lib.qfm_last_error()
    bad = qfm.Qf8ShexpW(p, None, p, p)
    assert lib.qf8_shexp_ex(C.byref(bad), p, p, p, p, p, p, None) == -1
    assert b"null" in lib.qfm_last_error()
