"""The FP8 lane-chunk format (ocho/amd_server/qf8_moe_fp8.hip:19-37,
:217-246): the oracle's E4M3 decode/encode and expert pack pinned against
torch's float8_e4m3fn, closed forms and a numpy restatement; then the
library's host packer (qf8_fp8_pack_expert) against the oracle, bit for bit."""
import ctypes as C

import numpy as np
import pytest

import _oracle as orc
import qfm

torch = pytest.importorskip("torch")


def _torch_f8_bits(v):
    return torch.tensor(np.asarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_every_code():
    tab = orc.f8_decode_table()
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    for b in range(256):
        if b & 0x7F == 0x7F:
            assert tab[b] == (480.0 if b == 0x7F else -480.0)   # no NaN in this format
        else:
            assert tab[b].view(np.uint32) == ref[b].view(np.uint32), b
    assert tab[0x7E] == 448.0 and tab[0x01] == 2.0 ** -9 and tab[0x08] == 2.0 ** -6
    assert np.signbit(tab[0x80]) and tab[0x80] == 0.0


def test_encode_round_trip_and_nearest_even():
    lib = orc.load()
    tab = orc.f8_decode_table()
    for b in range(256):
        if (b & 0x7F) < 0x78 or (b & 0x7F) == 0x7E:
            assert lib.orc_f8_encode(float(tab[b])) == b, b
        elif (b & 0x7F) != 0x7F:                       # 256 .. 416 are never emitted: they saturate
            assert lib.orc_f8_encode(float(tab[b])) == (b & 0x80) | 0x7E, b
    rng = np.random.default_rng(1)
    mag = np.exp2(rng.uniform(-6, 8, 20000)).astype(np.float32)        # normal range [2^-6, 2^8)
    mid = (tab[0x08:0x77].astype(np.float64) + tab[0x09:0x78]) / 2       # exact half-way points
    v = np.concatenate([mag, mid.astype(np.float32)])
    v = np.concatenate([v, -v])
    v = v[np.abs(v) < 240]                          # torch saturation differs above the largest code below 2^8
    ours = np.array([lib.orc_f8_encode(float(x)) for x in v], np.uint8)
    assert np.array_equal(ours, _torch_f8_bits(v))


def test_encode_closed_forms():
    lib = orc.load()
    enc = lambda x: lib.orc_f8_encode(float(np.float32(x)))
    # below 2^-9: signed zero (no rounding up to the smallest subnormal)
    assert enc(2.0 ** -10) == 0 and enc(0.99 * 2.0 ** -9) == 0 and enc(-(2.0 ** -10)) == 0x80
    # subnormals truncate: code = floor(|v| / 2^-9)
    for q in np.linspace(1.0, 7.99, 57):
        x = q * 2.0 ** -9
        assert enc(x) == int(np.floor(q)) and enc(-x) == 0x80 | int(np.floor(q))
    # from 2^8 up, and any carry into exponent 8, saturate to 0x7E (448)
    for x in (256.0, 300.0, 448.0, 1e9, 255.0, 248.0):
        assert enc(x) == 0x7E and enc(-x) == 0xFE
    assert enc(240.0) == 0x77 and enc(244.0) == 0x77          # 244 = half-way 240/256, 0x77 is even -> stays


def _random_expert(rng, rows, n_in):
    W = rng.integers(0, 256, (rows, n_in // 2), dtype=np.uint8)
    S = rng.integers(0, 256, (rows, n_in // 16), dtype=np.uint8)   # every scale byte, 0x7F and >= 0x80 included
    return W, S


def test_pack_numpy_restatement():
    rng = np.random.default_rng(2)
    rows, n_in, s2 = 24, 2048, np.float32(0.0137)
    W, S = _random_expert(rng, rows, n_in)
    W[3] = 0                                                           # an all-zero row: scale 1, codes 0
    w8, sc = orc.fp8_pack_expert(W, S, s2, rows, n_in)
    e2m1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    e, m = np.arange(256) >> 3, np.arange(256) & 7
    bs = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8) * np.exp2(e - 7.0)).astype(np.float32)
    nib = np.stack([W & 15, W >> 4], axis=2).reshape(rows, n_in)
    v = e2m1[nib] * (bs[np.repeat(S, 16, axis=1)] * s2)                # float32 throughout
    ch = n_in // 64
    mx = np.abs(v).reshape(rows, 64, ch).max(axis=2)
    scale = np.where(mx > 0, mx / np.float32(448), np.float32(1)).astype(np.float32)
    assert np.array_equal(sc.view(np.uint32), scale.view(np.uint32))
    lib = orc.load()
    q = v / np.repeat(scale, ch, axis=1)
    codes = np.array([lib.orc_f8_encode(float(x)) for x in q.ravel()], np.uint8).reshape(rows, n_in)
    assert np.array_equal(w8, codes)
    assert np.all(w8[3] == 0) and np.all(sc[3] == 1.0)
    # every nonzero chunk's maximum (448 to within an ulp after the division) is coded 0x7E
    top = (w8 & 0x7F).reshape(rows, 64, ch).max(axis=2)
    assert np.all(top[mx > 0] == 0x7E)


@pytest.mark.parametrize("rows,n_in", [(32, 2048), (16, 512), (8, 2560), (12, 640)])
def test_library_packer_matches_oracle(rows, n_in):
    lib = qfm.load()
    rng = np.random.default_rng(rows + n_in)
    W, S = _random_expert(rng, rows, n_in)
    ref_w, ref_s = orc.fp8_pack_expert(W, S, 0.02, rows, n_in)
    w8 = np.empty((rows, n_in), np.uint8)
    sc = np.empty((rows, 64), np.float32)
    assert lib.qf8_fp8_pack_expert(W.ctypes.data, S.ctypes.data, C.c_float(0.02), rows, n_in, w8.ctypes.data,
                                   sc.ctypes.data) == 0
    assert np.array_equal(w8, ref_w)
    assert np.array_equal(sc.view(np.uint32), ref_s.view(np.uint32))
    assert lib.qf8_fp8_pack_expert(W.ctypes.data, S.ctypes.data, C.c_float(0.02), rows, 100, w8.ctypes.data,
                                   sc.ctypes.data) == -1
    lib.qfm_last_error()
