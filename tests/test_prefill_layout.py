"""Host-only checks of the prefill workspace carve-up (no GPU).

pf_layout (qwen-3-ocho_amd/csrc/qfm_prefill_layout.h) is the single source of
the prefill workspace offsets: the launcher, the workspace sizing and the
workspace view all read it. These tests compile it on the host and replay it
for token counts 9..16384, both arena formats, both shapes, with and without
the shared expert, and gate/up / down tile widths 64..256, checking that

* the regions are 256-byte aligned, in order, disjoint and inside the total;
* every region holds what the kernels index in it (items, pairs, partials,
  row sums) for the worst routing the bound admits;
* k_pf_plan's m-tile count never exceeds the bound the work lists and the
  GEMM grids are sized for, over adversarial, uniform and skewed routings,
  and every work item it writes lies inside its group;
* the library's own qfm_workspace_bytes equals the layout with the tile
  widths it is built with.
"""
import ctypes as C
import os
import subprocess
import tempfile

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NREG = 23
NAMES = ["lg", "xnorm", "wnorm", "wb16", "sel", "wts", "gam", "ctr", "off", "blk", "items_gu", "items_dn",
         "p_tok", "p_slot", "p_wt", "hid", "part", "partk", "xsum", "hsum", "x16", "x16sum", "x16isc"]
BM, SLICES, PAIRS_PER_BLK = 128, 1, 4096
GU_I8, GU_F4, DN_I8 = 256, 256, 128           # the tile widths the library is built with


@pytest.fixture(scope="module")
def shim():
    d = tempfile.mkdtemp(prefix="pflayout")
    so = os.path.join(d, "libpflayout.so")
    subprocess.run(["g++", "-O1", "-std=c++17", "-shared", "-fPIC", "-o", so,
                    os.path.join(ROOT, "tests", "prefill_layout_shim.cpp")], check=True)
    lib = C.CDLL(so)
    lib.pf_layout_c.restype = C.c_int
    return lib


def layout(shim, T, H, I, E, K, has_sh, gu, dn):
    off = (C.c_ulonglong * NREG)()
    by = (C.c_ulonglong * NREG)()
    meta = (C.c_ulonglong * 6)()
    n = shim.pf_layout_c(T, H, I, E, K, int(has_sh), gu, dn, BM, SLICES, PAIRS_PER_BLK, off, by, meta)
    assert n == NREG
    return (np.array(off[:], np.int64), np.array(by[:], np.int64),
            dict(total=meta[0], P=meta[1], max_mt=meta[2], nt_gu=meta[3], nt_dn=meta[4], nblk=meta[5]))


def plan_items(counts, nt):
    """k_pf_plan's work list for group row counts `counts`: (group, row0, rows, n)
    per m-tile and n-tile, in the kernel's order."""
    mt = (counts + BM - 1) // BM
    first = np.concatenate([[0], np.cumsum(mt)[:-1]])
    mtot = int(mt.sum())
    items = []
    for m in range(mtot):
        g = int(np.searchsorted(first, m, side="right") - 1)     # last group whose first m-tile <= m
        row0 = (m - int(first[g])) * BM
        rows = min(BM, int(counts[g]) - row0)
        items.extend((g, row0, rows, n) for n in range(nt))
    return mtot, items


TS = [9, 10, 37, 100, 128, 129, 300, 1000, 4095, 4096, 8037, 8038, 8192, 16384]
SHAPES = [(2048, 512), (2560, 640)]


@pytest.mark.parametrize("H,I", SHAPES)
@pytest.mark.parametrize("has_sh", [True, False])
@pytest.mark.parametrize("gu,dn", [(GU_I8, DN_I8), (GU_F4, GU_F4), (128, 64), (256, 256), (512, 128), (128, 256)])
def test_regions_disjoint_and_sized(shim, H, I, has_sh, gu, dn):
    E, K = 512, 10
    for T in TS:
        off, by, m = layout(shim, T, H, I, E, K, has_sh, gu, dn)
        assert (off % 256 == 0).all(), T
        ends = off + by
        assert (ends[:-1] <= off[1:]).all(), (T, [NAMES[i] for i in np.nonzero(ends[:-1] > off[1:])[0]])
        assert ends[-1] <= m["total"]
        S = K + (1 if has_sh else 0)
        P = T * S
        assert m["P"] == P
        nt_gu, nt_dn = I // (gu // 2), H // dn
        assert (m["nt_gu"], m["nt_dn"]) == (nt_gu, nt_dn)
        assert m["max_mt"] % 8 == 0                       # the XCD tile maps cover [0, max_mt * nt) exactly
        need = dict(lg=SLICES * T * E * 4, sel=T * K * 4, wts=T * K * 4, ctr=32, off=(E + 2) * 4,
                    blk=m["nblk"] * E * 4, items_gu=m["max_mt"] * nt_gu * 16, items_dn=m["max_mt"] * nt_dn * 16,
                    p_tok=P * 4, p_slot=P * 4, p_wt=P * 4, hid=P * I * 2, part=P * H * 2, partk=P * (H // 64),
                    hsum=P * nt_gu * 4,
                    x16=T * H * 2, x16sum=T * 4, x16isc=T * 4, wb16=E * H * 2)
        for k, v in need.items():
            assert by[NAMES.index(k)] >= v, (T, k, by[NAMES.index(k)], v)
        assert m["nblk"] * PAIRS_PER_BLK >= T * K
        # the m-tile bound: every group of c rows needs ceil(c / BM) <= c / BM + 1 tiles
        assert m["max_mt"] >= P // BM + E + 1


def _routings(T, K, E, rng):
    """Per-expert routed counts (each token picks K distinct experts): uniform,
    skewed, and the adversary that maximizes m-tiles (BM + 1 rows per expert)."""
    out = []
    for skew in (0.0, 1.5, 4.0):
        p = np.exp(skew * rng.standard_normal(E))
        p /= p.sum()
        cnt = np.zeros(E, np.int64)
        for _ in range(T):
            cnt[rng.choice(E, K, replace=False, p=p)] += 1
        out.append(cnt)
    adv = np.zeros(E, np.int64)
    left = T * K
    for e in range(E):                                    # BM + 1 rows each while pairs last, never above T
        c = min(BM + 1, T, left)
        adv[e] = c
        left -= c
    if left > 0:                                          # the rest spread (count <= T per expert)
        for e in range(E):
            add = min(T - adv[e], left)
            adv[e] += add
            left -= add
    out.append(adv)
    return out


@pytest.mark.parametrize("H,I", SHAPES)
@pytest.mark.parametrize("gu,dn", [(GU_I8, DN_I8), (GU_F4, GU_F4), (128, 64), (256, 256)])
def test_plan_fits_the_bounds(shim, H, I, gu, dn):
    E, K = 512, 10
    rng = np.random.default_rng(5)
    for T in (9, 37, 300, 2000, 8038):
        for has_sh in (True, False):
            off, by, m = layout(shim, T, H, I, E, K, has_sh, gu, dn)
            for cnt in _routings(T, K, E, rng):
                assert cnt.sum() == T * K and cnt.max() <= T
                groups = np.concatenate([cnt, [T] if has_sh else []]).astype(np.int64)
                for nt, cap in ((m["nt_gu"], by[NAMES.index("items_gu")] // 16),
                                (m["nt_dn"], by[NAMES.index("items_dn")] // 16)):
                    mtot, items = plan_items(groups, nt)
                    assert mtot <= m["max_mt"], (T, mtot, m["max_mt"])
                    assert len(items) <= cap
                    for g, row0, rows, n in items:
                        assert 0 < rows <= BM and row0 + rows <= groups[g] and 0 <= n < nt


def test_library_sizes_match_the_layout(shim):
    """qfm_workspace_bytes (M > 8) = the workspace's tag header (256 bytes of row
    tags, 8 rows x E 8-byte logit words and 8 rows x (K + 1) slots x H 8-byte
    partial words, kept by the M <= 8 forward) + the larger of the INT8 and
    NVFP4 layouts with the shared expert, at the tile widths the library is
    built with."""
    import qfm
    lib = qfm.load()
    for H, I in SHAPES:
        hdr = 256 + 8 * 512 * 8 + 8 * 11 * H * 8
        qfm.init(H, I, 512, 10, 1, 1)
        for T in TS:
            a = layout(shim, T, H, I, 512, 10, True, GU_I8, DN_I8)[2]["total"]
            b = layout(shim, T, H, I, 512, 10, True, GU_F4, GU_F4)[2]["total"]
            assert lib.qfm_workspace_bytes(T) == hdr + max(a, b), (H, T)
    qfm.init(2048, 512, 512, 10, 1, 1)
