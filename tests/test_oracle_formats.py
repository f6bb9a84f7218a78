"""Pins of the CPU oracle's generator and number formats (no GPU).

Each check is independent of the oracle's own formulas: published KATs,
the reference's code tables, library conversions (torch's float8 / bfloat16
casts) and brute force.
"""
import json
import os

import numpy as np
import pytest

import _oracle as orc

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _hex(v):
    return int(v, 16)


def test_philox_kat():
    kat = json.load(open(os.path.join(GOLD, "philox_kat.json")))
    for v in kat["vectors"]:
        out = orc.philox([_hex(c) for c in v["ctr"]], [_hex(k) for k in v["key"]])
        assert [int(o) for o in out] == [_hex(o) for o in v["out"]]


def test_stream_word_mapping():
    # word j of (seed, layer, tensor) = word j%4 of philox(ctr=(j/4 lo, hi, tensor, layer), key=(seed,0))
    lib = orc.load()
    for seed, layer, tensor, j in [(0, 0, 1, 0), (7, 3, 2, 5), (1, 47, 8, (1 << 34) + 6), (0, 1, 16, 123456789)]:
        b = j >> 2
        blk = orc.philox([b & 0xFFFFFFFF, b >> 32, tensor, layer], [seed, 0])
        assert lib.orc_word(seed, layer, tensor, j) == int(blk[j & 3])


def test_gen_i8_range_and_uniformity():
    q = orc.fill("i8", 0, 0, orc.T_QG, 0, 255 * 4000)
    assert q.min() == -127 and q.max() == 127
    counts = np.bincount(q.astype(np.int64) + 127, minlength=255)
    exp = q.size / 255
    chi2 = ((counts - exp) ** 2 / exp).sum()
    assert chi2 < 254 + 6 * np.sqrt(2 * 254)   # ~6 sigma of a chi2(254)


def test_gen_i8_closed_form():
    lib = orc.load()
    for n in [0, 1, 2, 3, 17, 10 ** 6 + 3]:
        w = lib.orc_word(5, 2, orc.T_QD, n)
        assert lib.orc_gen_i8(5, 2, orc.T_QD, n) == ((w * 255) >> 32) - 127


def test_gen_rowscale_range_and_form():
    s = orc.fill("rowscale", 0, 1, orc.T_SG, 0, 100000)
    c = np.float32(0.02) / np.float32(127.0)
    assert s.min() >= 0.5 * c and s.max() < 1.5 * c
    lib = orc.load()
    for n in range(50):
        w = lib.orc_word(0, 1, orc.T_SG, n)
        u = (w >> 8) / 2.0 ** 24
        exact = (0.5 + u) * float(c)   # the fma computes this exactly before one rounding
        assert s[n] == np.float32(exact)


def test_gen_gauss_moments_and_form():
    z = orc.fill("gauss", 0, 0, orc.T_X, 0, 200000, 1.0)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert np.abs(z).max() <= 6.0
    lib = orc.load()
    for n in [0, 1, 999]:
        words = [lib.orc_word(0, 0, orc.T_X, 12 * n + i) for i in range(12)]
        s = sum(w >> 8 for w in words) - 6 * 2 ** 24
        assert z[n] == np.float32(s) / np.float32(2 ** 24)


def test_gen_fp4byte_and_scales():
    b = orc.fill("fp4byte", 0, 0, orc.T_FG, 0, 160000)
    lo, hi = b & 15, b >> 4
    for nib in (lo, hi):
        c = np.bincount(nib, minlength=16)
        assert c.min() > 0.9 * nib.size / 16
    sc = orc.fill("e4m3scale", 0, 0, orc.T_FSG, 0, 100000)
    lib = orc.load()
    vals = np.array([lib.orc_e4m3(int(v)) for v in np.unique(sc)])
    assert vals.min() >= 0.25 and vals.max() <= 2.0


def test_e2m1_table_matches_reference_lut():
    tab = json.load(open(os.path.join(GOLD, "nvfp4_tables.json")))["e2m1"]
    lib = orc.load()
    got = [lib.orc_e2m1(n) for n in range(16)]
    assert got == tab
    # sign bit: n and n|8 are negatives of each other, including -0
    for n in range(8):
        assert np.signbit(np.float32(lib.orc_e2m1(n | 8)))


def test_e4m3_all_codes_vs_torch_and_reference_formula():
    import torch
    lib = orc.load()
    tab = json.load(open(os.path.join(GOLD, "nvfp4_tables.json")))["e4m3_anchors"]
    for code, v in tab.items():
        got = lib.orc_e4m3(int(code))
        assert (np.isinf(got) if v == "inf" else got == v)
    codes = np.arange(0, 127, dtype=np.uint8)   # 0x7F is the reference's +inf (NaN in OCP fn)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([lib.orc_e4m3(int(c)) for c in codes], np.float32)
    assert np.array_equal(got, ref)
    # the reference's ue4m3f formula: e==0 -> m*2^-9 else (8+m)*2^(e-10)
    for c in range(127):
        e, m = c >> 3, c & 7
        f = m * 2.0 ** -9 if e == 0 else (8 + m) * 2.0 ** (e - 10)
        assert got[c] == f
    # bytes >= 0x80: the reference reads e = byte >> 3 (five bits), so these are
    # unsigned scales 2^9 .. 2^24 * 1.875, not the negative OCP codes
    for c in range(128, 256):
        e, m = c >> 3, c & 7
        assert lib.orc_e4m3(c) == np.float32((8 + m) * 2.0 ** (e - 10))
    assert lib.orc_e4m3(0x80) == 512.0 and lib.orc_e4m3(0xFF) == np.float32(1.875 * 2.0 ** 24)


def test_e4m3_encode_roundtrip_and_nearest():
    import torch
    lib = orc.load()
    for c in range(8, 127):   # normals
        assert lib.orc_e4m3_encode(lib.orc_e4m3(c)) == c
    rng = np.random.default_rng(0)
    v = (0.25 + 1.75 * rng.random(20000)).astype(np.float32)
    # ties: midpoints between neighbouring codes must round to even mantissa
    mids = np.array([(lib.orc_e4m3(c) + lib.orc_e4m3(c + 1)) / 2 for c in range(40, 64)], np.float32)
    v = np.concatenate([v, mids])
    got = np.array([lib.orc_e4m3_encode(float(a)) for a in v], np.uint8)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


def test_bf16_rne_vs_torch():
    import torch
    lib = orc.load()
    rng = np.random.default_rng(1)
    v = rng.standard_normal(4096).astype(np.float32) * np.float32(10.0) ** rng.integers(-20, 20, 4096)
    # halfway cases: low 16 bits exactly 0x8000 with odd and even upper parts
    bits = rng.integers(0, 2 ** 31, 512, dtype=np.uint64).astype(np.uint32) & np.uint32(0x7F7F0000) | np.uint32(0x8000)  # exponent < 0xFF
    v = np.concatenate([v, bits.view(np.float32), np.array([0.0, -0.0, np.inf, -np.inf], np.float32)])
    got = np.array([lib.orc_bf16_rne(float(a)) for a in v], np.uint16)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.uint16).numpy()
    assert np.array_equal(got, ref)
    # fill_gauss_bf16 == bf16(fill_gauss)
    z = orc.fill("gauss", 3, 4, orc.T_X, 100, 5000, 1.0)
    zb = orc.fill("gauss_bf16", 3, 4, orc.T_X, 100, 5000)
    assert np.array_equal(zb, torch.from_numpy(z).to(torch.bfloat16).view(torch.uint16).numpy())


def test_i8_quant_bf16_closed_forms_and_restatement():
    """orc_i8_quant_bf16 (qf8_dense_i8.hip:41-60): scale = absmax / 127, codes
    rint(w * (1/scale)) clamped; ties round to even, a zero row keeps scale 1."""
    def bf(vals):   # fp32 -> bf16 bits, nearest even (inputs here are finite)
        u = np.asarray(vals, np.float32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    K = 32
    rows = np.zeros((4, K), np.uint16)
    rows[0] = bf([127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5, 126.5] + [0.0] * (K - 9))   # scale exactly 1
    rows[1] = 0                                                                              # zero row
    rows[2] = bf(np.linspace(-3, 3, K))
    rows[3] = bf([-1e-3] + [5e-4] * (K - 1))
    q, s = orc.i8_quant_bf16(rows)
    assert s[0] == 1.0 and list(q[0, :9]) == [127, 2, 4, -2, -4, 0, 2, 0, 126]            # rint, not round
    assert s[1] == 1.0 and not q[1].any()
    assert q[2, 0] == -127 and q[2, -1] == 127 and q[3, 0] == -127
    rng = np.random.default_rng(4)
    W = bf(rng.standard_normal((64, 2048)) * 0.05)
    q, s = orc.i8_quant_bf16(W)
    w = orc.bf16_to_f32(W)
    amax = np.abs(w).max(axis=1)
    sc = np.where(amax > 0, amax / np.float32(127), np.float32(1)).astype(np.float32)
    inv = (np.float32(1) / sc).astype(np.float32)
    ref = np.clip(np.rint(w * inv[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(s.view(np.uint32), sc.view(np.uint32))
    assert np.array_equal(q, ref)
