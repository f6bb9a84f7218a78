"""Weight store reader (qf_store_open / qf_find) and the layer preflight, on
the CPU. The safetensors parser is pinned against the safetensors library in
both directions (files it writes are read here; files written here are read
by it); the manifest form against records packed field by field from the
reference's layout (ocho/amd_server/qwenflash.h:12-30)."""
import ctypes as C
import json
import os
import struct
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "qwen-3-ocho_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import qfm  # noqa: E402
import make_store as ms  # noqa: E402

torch = pytest.importorskip("torch")
st_torch = pytest.importorskip("safetensors.torch")
from safetensors import safe_open  # noqa: E402


def _open_rc(path):
    lib = qfm.load()
    s = qfm.QfStore()
    rc = lib.qf_store_open(C.byref(s), str(path).encode())
    msg = lib.qfm_last_error().decode()
    if rc == 0:
        lib.qf_store_close(C.byref(s))
    return rc, msg


def _lib_tensors():
    g = torch.Generator().manual_seed(3)
    return {
        "a.weight": torch.randn(5, 7, generator=g).to(torch.bfloat16),
        "a.weight_scale_2": torch.tensor(0.25, dtype=torch.float32),
        "a.input_scale": torch.tensor(2.0, dtype=torch.float32),
        "b.f32": torch.randn(3, 2, 4, generator=g),
        "c.u8": torch.randint(0, 256, (64,), generator=g, dtype=torch.uint8),
        "d.e4m3": torch.randint(0, 256, (4, 8), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn),
        "e.i64": torch.arange(6, dtype=torch.int64).reshape(2, 3),
        "f.f16": torch.randn(9, generator=g).to(torch.float16),
        "g.empty": torch.zeros(0, 4, dtype=torch.float32),
    }


def _raw(t):
    return t.contiguous().reshape(-1).view(torch.uint8).numpy().tobytes() if t.numel() else b""


def test_reads_what_the_safetensors_library_writes(tmp_path):
    ts = _lib_tensors()
    p = tmp_path / "one.safetensors"
    st_torch.save_file(ts, str(p), metadata={"format": "pt"})
    codes = {torch.bfloat16: "BF16", torch.float32: "F32", torch.uint8: "U8", torch.float8_e4m3fn: "F8_E4M3",
             torch.int64: "I64", torch.float16: "F16"}
    s = qfm.Store(p)
    assert s.names() == sorted(ts)                       # sorted by strcmp (ASCII names)
    for name, t in ts.items():
        e = s.find(name)
        assert e is not None, name
        assert e.rec.dtype == qfm.DTYPE_CODES[codes[t.dtype]]
        shape = list(t.shape)
        assert list(e.rec.ne) == (list(reversed(shape)) + [1] * 4)[:4]
        assert e.rec.nbytes == t.numel() * t.element_size()
        assert s.data(e) == _raw(t)
        assert e.rec.file_idx == 0
    w = s.find("a.weight")
    # companion scales of "a.weight": offsets of a.weight_scale_2 / a.input_scale
    assert w.rec.scale2_off == s.find("a.weight_scale_2").rec.data_off
    assert w.rec.input_off == s.find("a.input_scale").rec.data_off
    assert s.find("b.f32").rec.scale2_off == 0
    assert s.find("nope") is None and s.find("a.weigh") is None and s.find("") is None
    s.close()


def test_library_reads_what_make_store_writes(tmp_path):
    rng = np.random.default_rng(5)
    w = rng.integers(0, 256, (6, 10), dtype=np.uint8)
    h = rng.integers(0, 65536, (3, 4), dtype=np.uint16)
    f = rng.standard_normal(7).astype(np.float32)
    p = tmp_path / "mine.safetensors"
    ms.write_safetensors(str(p), [("w", "U8", w.shape, w), ("h", "BF16", h.shape, h), ("f", "F32", f.shape, f),
                                  ("s", "F32", (), np.float32(1.5).tobytes())], metadata={"format": "pt"})
    with safe_open(str(p), framework="pt") as fh:
        assert sorted(fh.keys()) == ["f", "h", "s", "w"]
        assert np.array_equal(fh.get_tensor("w").numpy(), w)
        assert np.array_equal(fh.get_tensor("h").view(torch.int16).numpy().view(np.uint16), h)
        assert np.array_equal(fh.get_tensor("f").numpy(), f)
        assert float(fh.get_tensor("s")) == 1.5
        assert fh.metadata() == {"format": "pt"}


def test_directory_of_shards_and_manifest_form_agree(tmp_path):
    ts = _lib_tensors()
    names = sorted(ts)
    d = tmp_path / "st"
    d.mkdir()
    st_torch.save_file({k: ts[k] for k in names[:4]}, str(d / "m-00001.safetensors"))
    st_torch.save_file({k: ts[k] for k in names[4:]}, str(d / "m-00002.safetensors"))
    (d / "notes.txt").write_text("not a shard")
    a = qfm.Store(d)
    assert a.st.n_shards == 2 and a.names() == names
    for k in names:
        assert a.data(a.find(k)) == _raw(ts[k])
        assert a.find(k).rec.file_idx == (0 if k in names[:4] else 1)
    shards = [str(d / "m-00001.safetensors"), str(d / "m-00002.safetensors")]
    ms.manifest_from_safetensors(str(tmp_path / "idx"), shards)
    b = qfm.Store(tmp_path / "idx")
    assert b.names() == names
    for k in names:
        ea, eb = a.find(k), b.find(k)
        assert (ea.rec.file_idx, ea.rec.dtype, list(ea.rec.ne), ea.rec.data_off, ea.rec.nbytes) == \
               (eb.rec.file_idx, eb.rec.dtype, list(eb.rec.ne), eb.rec.data_off, eb.rec.nbytes)
        assert b.data(eb) == _raw(ts[k])


def test_manifest_record_layout(tmp_path):
    # one record packed by hand, byte by byte, from the reference struct layout
    shard = tmp_path / "blob.bin"
    shard.write_bytes(bytes(range(256)) * 4)
    rec = bytearray(512)
    rec[:9] = b"x.weight\0"
    struct.pack_into("<II", rec, 256, 0, 3)                       # file_idx, dtype (U8)
    struct.pack_into("<4Q", rec, 264, 16, 2, 1, 1)                # ne
    struct.pack_into("<QQ", rec, 296, 100, 32)                    # data_off, nbytes
    struct.pack_into("<QQII", rec, 312, 7, 9, 0, 0)               # scale2_off, input_off, files
    assert bytes(rec) == ms.manifest_record("x.weight", 0, 3, [16, 2], 100, 32, scale2_off=7, input_off=9)
    ms.write_manifest(str(tmp_path / "m"), [str(shard)], [bytes(rec)])
    s = qfm.Store(tmp_path / "m")
    e = s.find("x.weight")
    assert (e.rec.dtype, list(e.rec.ne), e.rec.data_off, e.rec.nbytes, e.rec.scale2_off) == (3, [16, 2, 1, 1], 100, 32, 7)
    assert s.data(e) == bytes(range(100, 132))


def _st_file(path, header_obj=None, raw_header=None, data=b"", hdr_len=None):
    hb = raw_header if raw_header is not None else json.dumps(header_obj).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb) if hdr_len is None else hdr_len))
        f.write(hb)
        f.write(data)


@pytest.mark.parametrize("case", [
    "short", "hdr_len_past_end", "not_object", "bad_json", "past_end", "size_mismatch", "bad_dtype",
    "too_many_dims", "negative", "float_offset", "name_too_long", "missing_field"])
def test_malformed_safetensors_rejected(tmp_path, case):
    p = tmp_path / "bad.safetensors"
    ok = {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "hdr_len_past_end":
        _st_file(p, ok, data=b"\0" * 8, hdr_len=10 ** 6)
    elif case == "not_object":
        _st_file(p, raw_header=b"[1, 2]")
    elif case == "bad_json":
        _st_file(p, raw_header=b'{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]', data=b"\0" * 8)
    elif case == "past_end":
        _st_file(p, {"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, data=b"\0" * 8)
    elif case == "size_mismatch":
        _st_file(p, {"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, data=b"\0" * 8)
    elif case == "bad_dtype":
        _st_file(p, {"t": {"dtype": "Q4", "shape": [8], "data_offsets": [0, 8]}}, data=b"\0" * 8)
    elif case == "too_many_dims":
        _st_file(p, {"t": {"dtype": "U8", "shape": [1, 1, 1, 1, 8], "data_offsets": [0, 8]}}, data=b"\0" * 8)
    elif case == "negative":
        _st_file(p, raw_header=b'{"t": {"dtype": "U8", "shape": [8], "data_offsets": [-1, 7]}}', data=b"\0" * 8)
    elif case == "float_offset":
        _st_file(p, raw_header=b'{"t": {"dtype": "U8", "shape": [8], "data_offsets": [0.0, 8]}}', data=b"\0" * 8)
    elif case == "name_too_long":
        _st_file(p, {"n" * 300: {"dtype": "U8", "shape": [8], "data_offsets": [0, 8]}}, data=b"\0" * 8)
    elif case == "missing_field":
        _st_file(p, {"t": {"dtype": "U8", "shape": [8]}}, data=b"\0" * 8)
    rc, msg = _open_rc(p)
    assert rc == -5, (rc, msg)
    assert msg


def test_open_errors(tmp_path):
    assert _open_rc(tmp_path / "missing")[0] == -1
    (tmp_path / "empty").mkdir()
    assert _open_rc(tmp_path / "empty")[0] == -1
    # duplicate tensor across two shards
    d = tmp_path / "dup"
    d.mkdir()
    for i in range(2):
        ms.write_safetensors(str(d / f"s{i}.safetensors"), [("same", "U8", (4,), b"abcd")])
    rc, msg = _open_rc(d)
    assert rc == -5 and "duplicate" in msg
    # manifest: partial record, missing shard, entry past the shard end, name without NUL
    m = tmp_path / "m"
    shard = tmp_path / "blob.bin"
    shard.write_bytes(b"\0" * 64)
    ms.write_manifest(str(m), [str(shard)], [ms.manifest_record("a", 0, 3, [8], 0, 8)])
    assert _open_rc(m)[0] == 0
    with open(m / "manifest.bin", "ab") as f:
        f.write(b"\0" * 100)
    assert _open_rc(m)[0] == -2
    ms.write_manifest(str(m), [str(tmp_path / "nope.bin")], [ms.manifest_record("a", 0, 3, [8], 0, 8)])
    assert _open_rc(m)[0] == -3
    ms.write_manifest(str(m), [str(shard)], [ms.manifest_record("a", 0, 3, [8], 60, 8)])
    assert _open_rc(m)[0] == -5
    ms.write_manifest(str(m), [str(shard)], [ms.manifest_record("a", 1, 3, [8], 0, 8)])
    assert _open_rc(m)[0] == -5
    bad = bytearray(ms.manifest_record("a", 0, 3, [8], 0, 8))
    bad[:256] = b"z" * 256
    ms.write_manifest(str(m), [str(shard)], [bytes(bad)])
    assert _open_rc(m)[0] == -5
    # a store that failed to open is left closed (nothing to free, find finds nothing)
    lib = qfm.load()
    s = qfm.QfStore()
    assert lib.qf_store_open(C.byref(s), str(m).encode()) == -5
    assert lib.qfm_last_error().decode()            # reading clears the latch
    assert s.n_entries == 0 and s.n_shards == 0 and not s.entries
    assert not lib.qf_find(C.byref(s), b"a")


@pytest.fixture(scope="module")
def sparse_layer(tmp_path_factory):
    """A full-size layer-3 index at H=2048, I=512, E=512 with the data left as holes."""
    d = tmp_path_factory.mktemp("sparse")
    paths = ms.synthetic_layer(str(d), 2048, 512, 512, 3, 7, shards=3, sparse=True)
    return d, paths


def test_layer_preflight(sparse_layer):
    d, paths = sparse_layer
    qfm.init(hidden=2048, inter=512)
    lib = qfm.load()
    lib.qfm_last_error()                               # start from an empty latch
    s = qfm.Store(d)
    assert s.st.n_entries == 512 * 9 + 5
    assert lib.qfm_store_check_layer(C.byref(s.st), 3) == 0, lib.qfm_last_error().decode()
    assert lib.qfm_store_check_layer(C.byref(s.st), 4) == -1
    assert "layers.4.mlp.gate.weight" in lib.qfm_last_error().decode()
    # the same index under the other shape is mis-sized
    qfm.init(hidden=2560, inter=640)
    assert lib.qfm_store_check_layer(C.byref(s.st), 3) == -1
    assert "mis-sized" in lib.qfm_last_error().decode()
    qfm.init(hidden=2048, inter=512)


def test_layer_preflight_names_the_bad_expert_tensor(tmp_path):
    qfm.init(hidden=2048, inter=512)
    H, I, E, L = 2048, 512, 512, 0
    ts = []
    for e in range(E):
        t = ms.expert_tensors(L, e, H, I)
        if e == 311:   # down_proj block scales one row short
            t = [(n, dt, (H - 1, I // 16) if n.endswith("down_proj.weight_scale") else sh, dat) for n, dt, sh, dat in t]
        ts += t
    ts += ms.dense_tensors(L, H, I, E)
    ms.write_safetensors(str(tmp_path / "x.safetensors"), ts)
    s = qfm.Store(tmp_path / "x.safetensors")
    lib = qfm.load()
    lib.qfm_last_error()
    assert lib.qfm_store_check_layer(C.byref(s.st), L) == -1
    msg = lib.qfm_last_error().decode()
    assert "L0 E311 down_proj" in msg, msg


# ------------------------------------------------------------------ memory preflight pricing
def test_preflight_pricing_matches_the_reference_slot_sizes():
    """qfm_expcache_bytes / qfm_arena_bytes (priced before any allocation, the
    reference's budget guard qf_hip4_stage.hip:792-813) against the reference's
    own per-expert constants at 2560/640: QF5_EXP_SLOT_BYTES = 2,764,800
    (qf_nvfp4_wave64.h:67-69), QF8_FP8_SLOT_BYTES = 3*640*2560 + 2*640*64*4
    + 2560*64*4 (qf8_moe_fp8.h:38-39) and the INT8 slot 3*640*2560 +
    (2*640 + 2560)*4 = 4,930,560 (qf_hip4_stage.hip:808)."""
    lib = qfm.load()
    qfm.init(2560, 640, 512, 10, 1, 1)
    E, slots = 512, 192
    nv, fp8, i8 = 2764800, 3 * 640 * 2560 + 2 * 640 * 64 * 4 + 2560 * 64 * 4, 4930560
    routing = lambda S: E * 4 + S * 4 + S * 8 + 8 + 16 * 4 + 3 * E * 4
    NV, I8, RING, F8 = 1, 2, 4, 8
    assert lib.qfm_expcache_bytes(slots, NV) == slots * nv + routing(slots)
    assert lib.qfm_expcache_bytes(slots, NV | I8) == slots * (nv + i8) + routing(slots)
    assert lib.qfm_expcache_bytes(E, NV | I8 | RING) == 2 * nv + E * i8 + routing(E)
    assert lib.qfm_expcache_bytes(slots, F8) == slots * fp8 + routing(slots)
    for bad in ((slots, 0), (slots, F8 | NV), (slots, RING | NV), (0, NV), (E + 1, NV), (slots, 16)):
        assert lib.qfm_expcache_bytes(*bad) == 0, bad
    assert lib.qfm_arena_bytes(qfm.QFM_FMT_NVFP4) == E * nv + 3 * E * 4
    assert lib.qfm_arena_bytes(qfm.QFM_FMT_INT8) == E * i8
    assert lib.qfm_arena_bytes(7) == 0
    qfm.init(2048, 512, 512, 10, 1, 1)
    # one config-1 layer: 512 routed INT8 experts of 3,158,016 bytes; with the shared expert
    # and the fp32 router the layer is the 1,624,256,512 bytes of the benchmark's workload
    assert lib.qfm_arena_bytes(qfm.QFM_FMT_INT8) == 512 * 3158016
    assert lib.qfm_arena_bytes(qfm.QFM_FMT_INT8) + 3158016 + 512 * 2048 * 4 == 1624256512
    # the budget setter: 0 means no limit beyond the device
    old = lib.qfm_get_hbm_budget()
    assert lib.qfm_set_hbm_budget(123 << 20) == 0 and lib.qfm_get_hbm_budget() == 123 << 20
    lib.qfm_set_hbm_budget(old)
