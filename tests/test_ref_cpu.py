"""The reference's own code (oracle/_ref, compiled from the checkout) against
this library, on the CPU: the FP8 lane-chunk packer
(ocho/amd_server/qf8_moe_fp8.hip:217-246) and the store reader
(ocho/amd_server/reader.cpp) on a manifest index."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import _ref
import qfm

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_store as ms  # noqa: E402


@pytest.mark.parametrize("rows,n_in,s2", [(16, 2560, 0.01), (24, 640, 0.37), (8, 2560, 3e-5)])
def test_fp8_packer_matches_reference(rows, n_in, s2):
    ref = _ref.kernels()
    lib = qfm.load()
    rng = np.random.default_rng(rows + n_in)
    W = rng.integers(0, 256, (rows, n_in // 2), dtype=np.uint8)
    S = rng.integers(0, 256, (rows, n_in // 16), dtype=np.uint8)      # every scale byte, 0x7F and >= 0x80 included
    W[1] = 0
    outs = []
    for L in (ref, lib):
        w8 = np.empty((rows, n_in), np.uint8)
        sc = np.empty((rows, 64), np.float32)
        fn = L.qf8_fp8_pack_expert
        fn.restype = C.c_int
        fn.argtypes = [C.c_void_p, C.c_void_p, C.c_float, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        assert fn(W.ctypes.data, S.ctypes.data, s2, rows, n_in, w8.ctypes.data, sc.ctypes.data) == 0
        outs.append((w8, sc))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))


def test_store_reader_matches_reference(tmp_path):
    rd = _ref.reader()
    rng = np.random.default_rng(4)
    shards = []
    for i in range(2):
        ts = [(f"t{i}.{j:03d}", "U8", (int(rng.integers(1, 300)),), None) for j in range(40)]
        ts += [(f"model.language_model.layers.{i}.mlp.gate.weight", "BF16", (8, 16), None)]
        p = str(tmp_path / f"s{i}.safetensors")
        ms.write_safetensors(p, ts)
        shards.append(p)
    ms.manifest_from_safetensors(str(tmp_path / "idx"), shards)
    openf = getattr(rd, "_Z13qf_store_openP7QfStorePKc")
    findf = getattr(rd, "_Z7qf_findPK7QfStorePKc")
    closef = getattr(rd, "_Z14qf_store_closeP7QfStore")
    openf.restype, openf.argtypes = C.c_int, [C.POINTER(qfm.QfStore), C.c_char_p]
    findf.restype, findf.argtypes = C.POINTER(qfm.QfEntry), [C.POINTER(qfm.QfStore), C.c_char_p]
    closef.restype, closef.argtypes = None, [C.POINTER(qfm.QfStore)]
    rs = qfm.QfStore()
    assert openf(C.byref(rs), str(tmp_path / "idx").encode()) == 0
    mine = qfm.Store(tmp_path / "idx")
    assert rs.n_entries == mine.st.n_entries and rs.n_shards == mine.st.n_shards
    names = mine.names()
    assert [rs.entries[i].name.decode() for i in range(rs.n_entries)] == names
    for nm in names + ["absent", ""]:
        a = findf(C.byref(rs), nm.encode())
        b = mine.find(nm)
        assert bool(a) == (b is not None), nm
        if b is not None:
            ea = a.contents
            assert (ea.rec.file_idx, ea.rec.dtype, list(ea.rec.ne), ea.rec.data_off, ea.rec.nbytes) == \
                   (b.rec.file_idx, b.rec.dtype, list(b.rec.ne), b.rec.data_off, b.rec.nbytes)
    closef(C.byref(rs))
