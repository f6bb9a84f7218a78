"""The dense INT8 x X8 GEMV, hyper-connection norm / combine and stream
inject of the oracle (ocho/amd_server/qf8_dense_i8.hip:78-175,
qf8_hc.hip:99-103) pinned by numpy restatements and closed forms."""
import numpy as np

import _oracle as orc


def _x8(v):
    return orc.x8_quant(np.asarray(v, np.float32))


def test_i8_gemv_numpy_and_closed_forms():
    rng = np.random.default_rng(1)
    rows, K = 37, 640
    W = rng.integers(-127, 128, (rows, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.01, rows).astype(np.float32)
    xq, xs = _x8(rng.standard_normal(K).astype(np.float32))
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    ref = (W.astype(np.float64) @ xd) * s
    y0 = orc.i8_gemv(W, s, xq, xs, 0)
    assert np.allclose(y0, ref, rtol=1e-13, atol=1e-15)
    q = ref * 0.25
    assert np.allclose(orc.i8_gemv(W, s, xq, xs, 1), q / (1 + np.exp(-q)), rtol=1e-13)
    assert np.allclose(orc.i8_gemv(W, s, xq, xs, 2), 2 / (1 + np.exp(-q)), rtol=1e-13)
    # one-hot row: y = s * code * block scale
    W1 = np.zeros((1, K), np.int8)
    W1[0, 100] = 3
    assert orc.i8_gemv(W1, np.float32([0.5]), xq, xs, 0)[0] == 0.5 * 3 * int(xq[100]) * float(xs[100 // 32])
    # silu(0) = 0, 2 sigmoid(0) = 1
    z = np.zeros((2, K), np.int8)
    assert list(orc.i8_gemv(z, np.ones(2, np.float32), xq, xs, 1)) == [0.0, 0.0]
    assert list(orc.i8_gemv(z, np.ones(2, np.float32), xq, xs, 2)) == [1.0, 1.0]


def test_hc_norm_and_combine():
    rng = np.random.default_rng(2)
    H = 2560
    R = rng.standard_normal(H).astype(np.float32)
    w = np.zeros(H, np.uint16)                                  # bf16 zero: normed = R * rstd
    n = orc.hc_norm(R, w)
    r64 = R.astype(np.float64)
    assert np.allclose(n, r64 / np.sqrt(np.mean(r64 ** 2) + 1e-6), rtol=1e-14)
    wb = (np.float32(0.5).view(np.uint32) >> 16).astype(np.uint16)   # bf16 0.5: factor 1.5
    n2 = orc.hc_norm(R, np.full(H, wb, np.uint16))
    assert np.allclose(n2, 1.5 * n, rtol=1e-14)
    hcy = rng.standard_normal(4 * H).astype(np.float32)
    normed = rng.standard_normal(4 * H).astype(np.float32)
    mixed = orc.hc_combine(hcy, normed, H)
    sig = 1 / (1 + np.exp(-hcy.astype(np.float64)))
    ref = 0.25 * (sig * normed.astype(np.float64)).reshape(4, H).sum(axis=0)
    assert np.allclose(mixed, ref, rtol=1e-14, atol=1e-15)
    # four equal streams: the mean is the stream itself
    same = np.tile(hcy[:H], 4), np.tile(normed[:H], 4)
    assert np.allclose(orc.hc_combine(*same, H), sig[:H] * normed[:H], rtol=1e-14)


def test_stream_inject_is_one_fma():
    rng = np.random.default_rng(3)
    H = 2048
    # operands in [0.5, 2): the exact a*b + c spans < 53 bits, so fp64 holds it exactly
    R = rng.uniform(0.5, 2, 4 * H).astype(np.float32)
    y = rng.uniform(0.5, 2, H).astype(np.float32)
    inj = rng.uniform(0.5, 2, 4).astype(np.float32)
    got = orc.stream_inject(R, y, inj)
    exact = np.repeat(inj.astype(np.float64), H) * np.tile(y.astype(np.float64), 4) + R.astype(np.float64)
    assert np.array_equal(got, exact.astype(np.float32))
    two = (np.repeat(inj, H) * np.tile(y, 4)).astype(np.float32) + R       # two roundings differ somewhere
    assert not np.array_equal(got, two)
