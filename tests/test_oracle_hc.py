"""The dense INT8 x X8 GEMV, hyper-connection norm / combine, stream
inject and bf16 shared expert of the oracle (ocho/amd_server/qf8_dense_i8.hip:78-175,
qf8_hc.hip:99-103, qf8_layer.hip:23-54) pinned by numpy restatements and closed forms."""
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


def _bf16(a):
    """fp32 -> bf16 bits (round to nearest even), and the values they hold."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return b, (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def test_shexp_bf16_numpy_and_closed_forms():
    rng = np.random.default_rng(4)
    M, H, I = 3, 256, 64
    gb, g = _bf16(rng.standard_normal((I, H)) * 0.05)
    ub, u = _bf16(rng.standard_normal((I, H)) * 0.05)
    db, d = _bf16(rng.standard_normal((H, I)) * 0.05)
    ib, gi = _bf16(rng.standard_normal(H) * 0.05)
    x = rng.standard_normal((M, H)).astype(np.float32)
    y0 = rng.standard_normal((M, H)).astype(np.float32)
    eg, eu, g1, ed, y = orc.shexp_bf16(gb, ub, db, ib, x, y0)
    x64 = x.astype(np.float64)
    gg, uu, g1r = x64 @ g.T, x64 @ u.T, x64 @ gi
    egr = gg / (1 + np.exp(-gg)) * uu
    edr = egr @ d.T
    assert np.allclose(eu, uu, rtol=1e-12, atol=1e-14) and np.allclose(g1, g1r, rtol=1e-12, atol=1e-14)
    assert np.allclose(eg, egr, rtol=1e-12, atol=1e-14) and np.allclose(ed, edr, rtol=1e-12, atol=1e-14)
    assert np.allclose(y, y0 + edr / (1 + np.exp(-g1r))[:, None], rtol=1e-12, atol=1e-14)
    # one-hot rows: gate row r picks x[r], up row r picks x[r + 1], down row o picks eg[o mod I]
    G = np.zeros((I, H), np.float32); U = np.zeros((I, H), np.float32); D = np.zeros((H, I), np.float32)
    G[np.arange(I), np.arange(I)] = 1.0
    U[np.arange(I), np.arange(I) + 1] = 1.0
    D[np.arange(H), np.arange(H) % I] = 2.0
    zi = np.zeros(H, np.uint16)                                   # gate_inp 0: factor sigmoid(0) = 1/2
    eg1, eu1, g11, ed1, y1 = orc.shexp_bf16(_bf16(G)[0], _bf16(U)[0], _bf16(D)[0], zi, x, np.zeros((M, H)))
    xa, xb = x64[:, :I], x64[:, 1:I + 1]
    assert np.array_equal(eu1, xb) and np.array_equal(g11, np.zeros(M))
    assert np.allclose(eg1, xa / (1 + np.exp(-xa)) * xb, rtol=1e-15)
    assert np.allclose(y1, 0.5 * 2.0 * eg1[:, np.arange(H) % I], rtol=1e-15)
    # zero x: eg, ed = 0 and y unchanged
    _, _, _, edz, yz = orc.shexp_bf16(gb, ub, db, ib, np.zeros((M, H), np.float32), y0)
    assert not edz.any() and np.array_equal(yz, y0.astype(np.float64))
