"""Pins of the CPU oracle's router, top-k, experts, CSR and layer (no GPU).

Each oracle function is checked against something that does not retype
its formula: numpy fp64 matmuls of independently dequantized weights,
brute-force selection by a stable sort, exact-arithmetic special cases,
closed forms (one-hot weights) and structural invariants.
"""
import ctypes as C

import numpy as np
import pytest

import _oracle as orc

RNG = np.random.default_rng(1234)


def _bf16(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).view(torch.uint16).numpy()


# ---------------------------------------------------------------- router
@pytest.mark.parametrize("H", [2048, 2560])
def test_router_vs_fp64_within_bound(H):
    E, M = 64, 3
    W = (RNG.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = _bf16(RNG.standard_normal((M, H)))
    lg = orc.router_logits(W, x)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    ref = xf @ W.astype(np.float64).T
    absdot = np.abs(xf) @ np.abs(W.astype(np.float64)).T
    # canonical order: 32/40-term fma chains + 6 tree levels -> |err| <= (H/64 + 6) u sum|w x|
    bound = (H / 64 + 6 + 2) * 2.0 ** -24 * absdot
    assert np.all(np.abs(lg - ref) <= bound)


def test_router_exact_on_representable_inputs():
    # small integers scaled by powers of two: every product and partial sum is exact
    E, H, M = 32, 2048, 2
    W = RNG.integers(-8, 9, (E, H)).astype(np.float32) * np.float32(2.0 ** -6)
    xi = RNG.integers(-8, 9, (M, H)).astype(np.float32)
    x = _bf16(xi)
    lg = orc.router_logits(W, x)
    ref = xi.astype(np.float64) @ W.astype(np.float64).T
    assert np.array_equal(lg.astype(np.float64), ref)
    bias = RNG.integers(-4, 5, E).astype(np.float32)
    lgb = orc.router_logits(W, x, bias)
    assert np.array_equal(lgb.astype(np.float64), ref + bias)


def test_router_canonical_order_is_the_documented_one():
    # Numpy restatement of the documented order with exactly-rounded fma emulated
    # through Python fractions on a small case (one row).
    from fractions import Fraction
    H = 256
    w = (RNG.standard_normal(H) * 0.02).astype(np.float32)
    x = _bf16(RNG.standard_normal(H))
    xf = orc.bf16_to_f32(x)

    def rnd(fr):   # correctly rounded Fraction -> float32, ties to even
        f = np.float32(float(fr))
        cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
        best = min(cands, key=lambda c: (abs(Fraction(float(c)) - fr), int(np.array(c).view(np.uint32)) & 1))
        return np.float32(best)

    p = []
    for l in range(64):
        a = np.float32(0.0)
        for j in range(H // 256):
            for c in range(4):
                k = j * 256 + 4 * l + c
                a = rnd(Fraction(float(w[k])) * Fraction(float(xf[k])) + Fraction(float(a)))
        p.append(a)
    p = np.array(p, np.float32)
    for m in (1, 2, 4, 8, 16, 32):
        p = (p + p[np.arange(64) ^ m]).astype(np.float32)
    lg = orc.router_logits(w[None, :], x[None, :])
    assert lg[0, 0] == p[0]


# ---------------------------------------------------------------- top-k
def _brute_topk(lg, K):
    # descending value, ties -> lower index: stable sort on -value
    return np.argsort(-lg, axis=-1, kind="stable")[:, :K]


def test_topk_matches_brute_force_and_softmax():
    from scipy.special import softmax
    M, E, K = 64, 512, 10
    lg = (RNG.standard_normal((M, E)) * 0.9).astype(np.float32)
    sel, w64, w32 = orc.topk(lg, K, renorm=1)
    assert np.array_equal(sel, _brute_topk(lg, K))
    p = softmax(lg.astype(np.float64), axis=-1)
    ps = np.take_along_axis(p, sel, axis=-1)
    assert np.allclose(w64, ps / ps.sum(-1, keepdims=True), rtol=1e-12, atol=0)
    assert np.allclose(w64.sum(-1), 1.0, rtol=1e-14)
    _, w64n, _ = orc.topk(lg, K, renorm=0)
    assert np.allclose(w64n, ps, rtol=1e-12)


@pytest.mark.parametrize("case", ["all_equal", "dup_boundary", "two_level", "quantized", "negzero"])
def test_topk_tie_catalogue(case):
    E, K = 512, 10
    if case == "all_equal":
        lg = np.zeros((1, E), np.float32)
    elif case == "dup_boundary":            # 9th..14th share one value: lower indices win
        lg = (RNG.standard_normal((1, E)) * 0.1).astype(np.float32)
        top = np.argsort(-lg[0])[:20]
        lg[0, top[8:14]] = lg[0, top[8]]
    elif case == "two_level":               # two groups of equal values straddling K
        lg = np.full((1, E), -1.0, np.float32)
        lg[0, [500, 3, 250, 7]] = 2.0
        lg[0, [9, 400, 1, 300, 100, 200, 2, 450]] = 1.0
    elif case == "quantized":               # few distinct levels everywhere
        lg = RNG.integers(0, 4, (4, E)).astype(np.float32)
    else:                                   # -0.0 and +0.0 compare equal: index decides
        lg = np.full((1, E), -5.0, np.float32)
        lg[0, [30, 10, 20]] = [-0.0, 0.0, -0.0]
        lg[0, 40] = 1.0
    sel, w64, _ = orc.topk(lg, K)
    assert np.array_equal(sel, _brute_topk(lg, K))
    assert np.allclose(w64.sum(-1), 1.0)
    if case == "all_equal":
        assert list(sel[0]) == list(range(K)) and np.allclose(w64, 1.0 / K)


# ---------------------------------------------------------------- experts
def _i8_expert_inputs(H, I):
    Qg = RNG.integers(-127, 128, (I, H)).astype(np.int8)
    Qu = RNG.integers(-127, 128, (I, H)).astype(np.int8)
    Qd = RNG.integers(-127, 128, (H, I)).astype(np.int8)
    sg = (RNG.random(I) + 0.5).astype(np.float32) * np.float32(0.02 / 127)
    su = (RNG.random(I) + 0.5).astype(np.float32) * np.float32(0.02 / 127)
    sd = (RNG.random(H) + 0.5).astype(np.float32) * np.float32(0.02 / 127)
    return Qg, sg, Qu, su, Qd, sd


def _silu(g):
    return g / (1.0 + np.exp(-g))


@pytest.mark.parametrize("H,I", [(2048, 512), (2560, 640)])
def test_i8_expert_vs_numpy(H, I):
    Qg, sg, Qu, su, Qd, sd = _i8_expert_inputs(H, I)
    x = orc.bf16_to_f32(_bf16(RNG.standard_normal(H))).astype(np.float64)
    h, y = orc.i8_expert(x, Qg, sg, Qu, su, Qd, sd)
    g = (Qg.astype(np.float64) * sg[:, None].astype(np.float64)) @ x
    u = (Qu.astype(np.float64) * su[:, None].astype(np.float64)) @ x
    href = _silu(g) * u
    yref = (Qd.astype(np.float64) * sd[:, None].astype(np.float64)) @ href
    assert np.allclose(h, href, rtol=1e-12, atol=1e-300)
    assert np.allclose(y, yref, rtol=1e-10, atol=1e-12 * np.abs(yref).max())


def test_i8_expert_closed_forms():
    H, I = 2048, 512
    # one-hot rows: gate row r picks x[r], up row r picks x[r+1], down row c picks h[c % I]
    Qg = np.zeros((I, H), np.int8); Qg[np.arange(I), np.arange(I)] = 1
    Qu = np.zeros((I, H), np.int8); Qu[np.arange(I), np.arange(I) + 1] = 2
    Qd = np.zeros((H, I), np.int8); Qd[np.arange(H), np.arange(H) % I] = -3
    sg = np.full(I, 0.5, np.float32); su = np.full(I, 0.25, np.float32); sd = np.full(H, 2.0, np.float32)
    x = np.linspace(-3, 3, H)
    h, y = orc.i8_expert(x, Qg, sg, Qu, su, Qd, sd)
    g = 0.5 * x[:I]; u = 0.5 * x[1:I + 1]
    assert np.allclose(h, g / (1 + np.exp(-g)) * u, rtol=1e-15)
    assert np.allclose(y, -6.0 * h[np.arange(H) % I], rtol=1e-15)
    h0, y0 = orc.i8_expert(np.zeros(H), *_i8_expert_inputs(H, I))
    assert not h0.any() and not y0.any()


def _nvfp4_dequant_numpy(F, S, s2, rows, K):
    tab = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])
    nib = np.empty((rows, K), np.int64)
    nib[:, 0::2] = F & 15
    nib[:, 1::2] = F >> 4
    e = (S >> 3).astype(np.int64); m = (S & 7).astype(np.int64)
    sc = np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10))
    return tab[nib] * np.repeat(sc, 16, axis=1) * float(np.float32(s2))


def test_nvfp4_dequant_and_expert_vs_numpy():
    H, I = 2048, 512
    Fg = RNG.integers(0, 256, (I, H // 2), dtype=np.uint8)
    Fu = RNG.integers(0, 256, (I, H // 2), dtype=np.uint8)
    Fd = RNG.integers(0, 256, (H, I // 2), dtype=np.uint8)
    Sg = RNG.integers(40, 65, (I, H // 16), dtype=np.uint8)
    Su = RNG.integers(40, 65, (I, H // 16), dtype=np.uint8)
    Sd = RNG.integers(0, 127, (H, I // 16), dtype=np.uint8)
    wg = _nvfp4_dequant_numpy(Fg, Sg, 0.01, I, H)
    assert np.array_equal(orc.nvfp4_dequant(Fg, Sg, 0.01, I, H), wg)
    x = orc.bf16_to_f32(_bf16(RNG.standard_normal(H))).astype(np.float64)
    h, y = orc.nvfp4_expert(x, Fg, Sg, 0.01, Fu, Su, 0.01, Fd, Sd, 0.01, H, I)
    wu = _nvfp4_dequant_numpy(Fu, Su, 0.01, I, H)
    wd = _nvfp4_dequant_numpy(Fd, Sd, 0.01, H, I)
    g = wg @ x; u = wu @ x
    href = _silu(g) * u
    assert np.allclose(h, href, rtol=1e-12, atol=1e-300)
    assert np.allclose(y, wd @ href, rtol=1e-10, atol=1e-12 * np.abs(wd @ href).max())


def test_nvfp4_nibble_order_ramp():
    # adjacent pairs: byte i = element 2i (low) | element 2i+1 (high)
    K = 32
    codes = np.arange(K) % 16
    F = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)[None, :]
    S = np.full((1, K // 16), 56, np.uint8)        # scale 1.0
    d = orc.nvfp4_dequant(F, S, 1.0, 1, K)[0]
    tab = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6])
    assert np.array_equal(d, tab[codes])


# ---------------------------------------------------------------- X8, CSR
def test_x8_quant_properties():
    v = (RNG.standard_normal(2048) * 3).astype(np.float32)
    v[64:96] = 0.0
    q, s = orc.x8_quant(v)
    assert np.abs(q.astype(int)).max() <= 127
    blocks = v.reshape(-1, 32)
    amax = np.abs(blocks).max(1)
    assert np.array_equal(s, np.where(amax > 0, amax * np.float32(1 / 127), 1).astype(np.float32))
    assert np.all(np.abs(q.reshape(-1, 32) * s[:, None] - blocks) <= 0.5 * s[:, None] * (1 + 1e-6))
    assert not q[64:96].any()


def test_m8_reduce4_exact_and_order():
    """orc_m8_reduce4 (qf_moe_m8_wave64.hip:216-221): y0 + y1 + y2 + y3 left to right in fp32."""
    rng = np.random.default_rng(5)
    ys = [rng.integers(-2 ** 20, 2 ** 20, 4099).astype(np.float32) for _ in range(4)]
    exact = sum(v.astype(np.int64) for v in ys)                     # every partial sum < 2^24: exact
    assert np.array_equal(orc.m8_reduce4(*ys), exact.astype(np.float32))
    # 2^24 + 1 + 1 + 1 left to right stays 2^24 (each +1 is a tie, to even); every
    # other association of the four gives 2^24 + 2 or 2^24 + 4, and the reversed
    # order 1 + 1 + 1 + 2^24 gives 2^24 + 4
    big, one = np.float32([2 ** 24]), np.float32([1.0])
    assert orc.m8_reduce4(big, one, one, one)[0] == 2 ** 24
    assert orc.m8_reduce4(one, one, one, big)[0] == 2 ** 24 + 4
    z = np.zeros(0, np.float32)
    assert orc.m8_reduce4(z, z, z, z).size == 0


def test_csr_invariants_and_order():
    T, K, E = 257, 10, 512
    sel = np.stack([RNG.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    wt = RNG.random((T, K)).astype(np.float32)
    ids, ptr, tok, kk, pw = orc.csr_build(sel, wt, E)
    assert np.all(np.diff(ids) > 0)
    assert ptr[0] == 0 and ptr[-1] == T * K and np.all(np.diff(ptr) > 0)
    order = np.argsort(sel.reshape(-1), kind="stable")           # (expert, token, k) order
    assert np.array_equal(tok, order // K) and np.array_equal(kk, order % K)
    assert np.array_equal(pw, wt.reshape(-1)[order])
    for i, e in enumerate(ids):
        seg = slice(ptr[i], ptr[i + 1])
        assert np.all(sel[tok[seg], kk[seg]] == e)
    with pytest.raises(ValueError):
        bad = sel.copy(); bad[3, 2] = E
        orc.csr_build(bad, wt, E)


# ---------------------------------------------------------------- layer
def test_layer_composes_the_pieces():
    H, I, E, K, M = 2048, 512, 64, 4, 2
    out = orc.moe_layer(H, I, E, K, M, seed=3, layer=5, x_layer=9, gated=1)
    x = out["x"]
    assert np.array_equal(x, orc.fill("gauss_bf16", 3, 9, orc.T_X, 0, M * H).reshape(M, H))
    W = orc.fill("gauss", 3, 5, orc.T_ROUTER, 0, E * H, 0.02).reshape(E, H)
    assert np.array_equal(out["logits"], orc.router_logits(W, x))
    sel, w64, _ = orc.topk(out["logits"], K)
    assert np.array_equal(out["sel"], sel)
    xf = orc.bf16_to_f32(x).astype(np.float64)

    def expert(e):
        Qg = orc.fill("i8", 3, 5, orc.T_QG, e * I * H, I * H).reshape(I, H)
        Qu = orc.fill("i8", 3, 5, orc.T_QU, e * I * H, I * H).reshape(I, H)
        Qd = orc.fill("i8", 3, 5, orc.T_QD, e * H * I, H * I).reshape(H, I)
        sg = orc.fill("rowscale", 3, 5, orc.T_SG, e * I, I)
        su = orc.fill("rowscale", 3, 5, orc.T_SU, e * I, I)
        sd = orc.fill("rowscale", 3, 5, orc.T_SD, e * H, H)
        return Qg, sg, Qu, su, Qd, sd

    g = orc.fill("gauss", 3, 5, orc.T_SHGATE, 0, H, 0.02).astype(np.float64)
    for m in range(M):
        y = np.zeros(H)
        for k in range(K):
            Qg, sg, Qu, su, Qd, sd = expert(sel[m, k])
            hh = _silu((Qg * sg[:, None].astype(np.float64)) @ xf[m]) * ((Qu * su[:, None].astype(np.float64)) @ xf[m])
            y += w64[m, k] * ((Qd * sd[:, None].astype(np.float64)) @ hh)
        Qg, sg, Qu, su, Qd, sd = expert(E)
        hh = _silu((Qg * sg[:, None].astype(np.float64)) @ xf[m]) * ((Qu * su[:, None].astype(np.float64)) @ xf[m])
        y += (1 / (1 + np.exp(-(g @ xf[m])))) * ((Qd * sd[:, None].astype(np.float64)) @ hh)
        assert np.allclose(out["y"][m], y, rtol=1e-9, atol=1e-12 * np.abs(y).max())
    assert np.array_equal(out["ybf"], _bf16(out["y"].astype(np.float32)))


# ---------------------------------------------------------------- NVFP4 -> INT8 build
def test_nvfp4_to_i8_closed_forms():
    K = 2048
    rows = 6
    F = RNG.integers(0, 256, (rows, K // 2), dtype=np.uint8)
    S = RNG.integers(40, 65, (rows, K // 16), dtype=np.uint8)
    F[1] = 0                                   # all-zero row: scale 1, codes 0
    F[2] = 0x22                                # every code 1.0 with a unit scale: constant row
    S[2] = 56
    F[3, 0] = 0x07                             # a +6 code (the row maximum at element 0)
    S[3, 0] = 63                               # largest scale in the row
    S[3, 1:] = np.minimum(S[3, 1:], 62)
    q, sc = orc.nvfp4_to_i8(F, S, 0.01, rows, K)
    v = orc.nvfp4_dequant(F, S, 0.01, rows, K)
    assert sc[1] == 1.0 and not q[1].any()
    assert np.all(q[2] == 127) and sc[2] == np.float32(np.float32(0.01) * np.float32(1 / 127))
    assert q[3, 0] == 127
    for r in range(rows):
        if r == 1:
            continue
        amax = np.abs(v[r]).max()
        assert abs(sc[r] - amax / 127) <= 2e-7 * sc[r]
        assert np.abs(q[r]).max() == 127
        # rint of the fp32 product v * (1/scale): within half a code plus the rounding of that product
        assert np.all(np.abs(q[r] * np.float64(sc[r]) - v[r]) <= (0.5 + 1e-5) * sc[r])
    # sign symmetry: flipping every code's sign bit negates every output code
    q2, sc2 = orc.nvfp4_to_i8(F ^ 0x88, S, 0.01, rows, K)
    assert np.array_equal(sc2, sc)
    assert np.array_equal(q2.astype(int), -q.astype(int))
    # the scale byte's exponent field is five bits wide: 0x80 | b reads as exponent >= 16
    F1 = np.full((1, 32), 0x22, np.uint8)
    S1 = np.array([[0x80 | 56, 56, 56, 56]], np.uint8)   # byte 0xB8: exponent 23 -> 2^16; the rest 1.0
    q1, s1 = orc.nvfp4_to_i8(F1, S1, 1.0, 1, 64)
    assert s1[0] == np.float32(np.float32((1 + 0 / 8) * 2.0 ** 16) * np.float32(1 / 127))
    assert np.all(q1[0, :16] == 127) and np.all(q1[0, 16:] == 0)


def test_x8_exact_ties_round_half_to_even():
    """X8 uses rintf (ties to even, qf8_moe_i8.hip:66), not roundf (ties away).
    With absmax 127 the scale is exactly 1.0 (fl(127 * fl(1/127)) = 1), so
    v = k + 1/2 lands exactly on a tie."""
    v = np.zeros(64, np.float32)
    v[0] = 127.0
    ties = np.array([0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, 126.5, -126.5, 5.5, 6.5, -7.5], np.float32)
    v[1:1 + ties.size] = ties
    v[32] = -127.0                                    # second block: absmax 127 again, negative
    v[33:33 + ties.size] = -ties
    q, s = orc.x8_quant(v)
    assert s[0] == 1.0 and s[1] == 1.0
    want = np.rint(ties).astype(np.int32)            # numpy rounds half to even
    assert np.array_equal(q[1:1 + ties.size], want)
    assert np.array_equal(q[33:33 + ties.size], -want)
    away = np.sign(ties) * np.floor(np.abs(ties) + 0.5)
    assert not np.array_equal(want, away)            # the case separates the two rules
    assert q[0] == 127 and q[32] == -127


@pytest.mark.parametrize("fmt,bias,renorm,gated", [(0, 1, 1, 1), (1, 1, 1, 1), (0, 0, 0, 0), (1, 0, 0, 1)])
def test_grouped_layer_matches_per_token_oracle(fmt, bias, renorm, gated):
    """The expert-grouped fp64 layer (the checker used for all 8038 prefill
    tokens) reproduces orc_moe_layer's per-token evaluation."""
    H, I, E, K, M = 2048, 512, 512, 10, 8
    r = orc.moe_layer(H, I, E, K, M, 4, 6, 60, fmt=fmt, use_bias=bias, renorm=renorm, gated=gated)
    g = orc.moe_layer_grouped(H, I, E, K, M, 4, 6, 60, fmt=fmt, use_bias=bias, renorm=renorm, gated=gated)
    assert np.array_equal(g["x"], r["x"])
    assert np.array_equal(g["sel"], r["sel"])
    assert np.array_equal(g["w"], r["w"])
    rel = np.abs(g["y"] - r["y"]).max() / np.abs(r["y"]).max()
    assert rel < 1e-12, rel


def test_cpu_baseline_path_matches_oracle():
    """orc_cpu_moe_layer_fast (the fp32 path bench.py times as the CPU baseline)
    against the fp64 oracle layer on the same generated layer: identical
    routing, outputs within the parity bound."""
    H, I, E, K, M, seed, layer, xl = 2048, 512, 512, 10, 3, 0, 5, 1005
    lib = orc.load()
    r = orc.moe_layer(H, I, E, K, M, seed, layer, xl)
    router = orc.fill("gauss", seed, layer, orc.T_ROUTER, 0, E * H, 0.02)
    g = orc.fill("gauss", seed, layer, orc.T_SHGATE, 0, H, 0.02)
    qg = np.zeros((E + 1) * I * H, np.int8); qu = np.zeros_like(qg); qd = np.zeros_like(qg)
    sg = np.zeros((E + 1) * I, np.float32); su = np.zeros_like(sg); sd = np.zeros((E + 1) * H, np.float32)
    for e in sorted(set(r["sel"].ravel().tolist())) + [E]:
        Qg, s_g, Qu, s_u, Qd, s_d = orc._i8_expert_arrays(seed, layer, e, H, I)
        qg[e * I * H:(e + 1) * I * H] = Qg.ravel(); qu[e * I * H:(e + 1) * I * H] = Qu.ravel()
        qd[e * H * I:(e + 1) * H * I] = Qd.ravel()
        sg[e * I:(e + 1) * I] = s_g; su[e * I:(e + 1) * I] = s_u; sd[e * H:(e + 1) * H] = s_d
    hl = orc.HostLayer(router.ctypes.data, qg.ctypes.data, qu.ctypes.data, qd.ctypes.data,
                       sg.ctypes.data, su.ctypes.data, sd.ctypes.data, g.ctypes.data)
    y = np.empty((M, H), np.float32)
    x = np.ascontiguousarray(r["x"])
    lib.orc_cpu_moe_layer_fast(C.byref(hl), H, I, E, K, x.ctypes.data, M, y.ctypes.data, 4)
    for m in range(M):
        rel = np.abs(y[m] - r["y"][m]).max() / np.abs(r["y"][m]).max()
        assert rel <= 1e-2, (m, rel)
        assert rel < 1e-4, (m, rel)                  # fp32 accumulation: far inside the bound
