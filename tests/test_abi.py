"""C-ABI checks that need no GPU: the library loads, exports every entry
point the headers under include/ declare, and the FFI struct layouts agree."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]
LIB = os.path.join(ROOT, "qwen-3-ocho_amd", "libqfm.so")


def _declared_functions():
    src = "\n".join(open(h).read() for h in HEADERS)
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    names = set()
    for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b([a-z_][A-Za-z0-9_]*)\s*\(", src, flags=re.M):
        name = m.group(1)
        if name not in ("if", "while", "for", "sizeof", "typedef"):
            names.add(name)
    return names


def _exported():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], check=True, capture_output=True, text=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}


@pytest.fixture(scope="module")
def built():
    if not os.path.exists(LIB):
        pytest.fail("libqfm.so not built: run __graft_entry__.build()")
    return LIB


def test_header_declares_expected_reference_entry_points():
    names = _declared_functions()
    for ref_name in ["qf_rtr_gemv_launch", "qf_rtr_topk10_launch", "qf_rtr_topk10_rows_launch",
                     "qf8_i8_gateup_m1", "qf8_i8_down_m1"]:
        assert ref_name in names


def test_every_declared_symbol_is_exported(built):
    declared = _declared_functions()
    exported = _exported()
    missing = sorted(declared - exported)
    assert not missing, f"declared but not exported: {missing}"
    # nothing beyond the header leaks out of the library
    extra = sorted(n for n in exported - declared if not n.startswith("_"))
    assert not extra, f"exported but not declared: {extra}"


def test_python_binding_covers_the_header(built):
    import qfm
    assert set(qfm.exported_symbols()) == _declared_functions()


def test_library_loads_without_gpu_and_struct_sizes_match(built):
    import qfm
    lib = qfm.load()
    assert lib.qfm_version().startswith(b"qfm")
    assert lib.qfm_sizeof(0) == C.sizeof(qfm.Qf4ExpCache) == 312
    assert lib.qfm_sizeof(1) == C.sizeof(qfm.QfmLayer)
    assert lib.qfm_sizeof(2) == C.sizeof(qfm.QfmSynthLayer)
    assert lib.qfm_sizeof(3) == C.sizeof(qfm.Qf8I8Mat) == 24
    assert lib.qfm_sizeof(4) == C.sizeof(qfm.Qf5M8Route) == 56
    assert lib.qfm_sizeof(5) == C.sizeof(qfm.QfmConfig)
    assert lib.qfm_sizeof(6) == C.sizeof(qfm.QfmWsView)
    assert lib.qfm_sizeof(7) == C.sizeof(qfm.QfEntry) == 512
    assert lib.qfm_sizeof(8) == C.sizeof(qfm.QfStore) == 56
    assert lib.qfm_sizeof(9) == C.sizeof(qfm.Qf4ExpXfer) == 48
    assert lib.qfm_sizeof(10) == C.sizeof(qfm.QfRouteMailbox) == 136
    # reference field offsets of the arena (qf_nvfp4_wave64.h:133-173 on LP64)
    assert qfm.Qf4ExpCache.i8_gate.offset == 80 and qfm.Qf4ExpCache.s_gate.offset == 136
    assert qfm.Qf4ExpCache.s2g_dev.offset == 256 and qfm.Qf4ExpCache.expected_seq.offset == 304


def test_config_validation_without_gpu(built):
    import qfm
    lib = qfm.load()
    bad = qfm.QfmConfig(2048, 640, 512, 10, 1, 1)
    assert lib.qfm_init(C.byref(bad)) != 0
    assert b"unsupported" in lib.qfm_last_error()
    assert lib.qfm_last_error() == b""              # reading clears the latch
    for cfg in [(2048, 512, 512, 10, 1, 1), (2560, 640, 512, 10, 1, 1), (2048, 512, 512, 4, 0, 0)]:
        c = qfm.QfmConfig(*cfg)
        assert lib.qfm_init(C.byref(c)) == 0
        out = qfm.QfmConfig()
        lib.qfm_get_config(C.byref(out))
        assert (out.hidden, out.inter, out.n_experts, out.top_k) == cfg[:4]
    assert lib.qfm_init(C.byref(qfm.QfmConfig(2048, 512, 512, 17, 1, 1))) != 0
    lib.qfm_last_error()
    # every path is built for the reference's 512 experts: other counts are rejected
    for e in (64, 256, 1024):
        assert lib.qfm_init(C.byref(qfm.QfmConfig(2048, 512, e, 4, 1, 1))) != 0
        assert b"unsupported" in lib.qfm_last_error()
    lib.qfm_init(C.byref(qfm.QfmConfig(2048, 512, 512, 10, 1, 1)))


def test_argument_rejection_without_gpu(built):
    import qfm
    lib = qfm.load()
    lib.qfm_init(C.byref(qfm.QfmConfig(2048, 512, 512, 10, 1, 1)))
    assert lib.qfm_moe_forward(None, None, 1, None, None, 0, None) != 0
    assert b"bad arguments" in lib.qfm_last_error()
    assert lib.qfm_router_logits(None, None, None, 1, None, None) != 0
    lib.qfm_last_error()
    assert lib.qfm_gen_fill(None, 0, 0, 10, 0, 0, 1, 0.0, None) != 0
    lib.qfm_last_error()
    assert lib.qfm_workspace_bytes(1) > 0 and lib.qfm_workspace_bytes(0) == 0


def test_validated_twins_reject_without_launching(built):
    """Every reference-named void launcher has an _ex twin returning a code; bad
    arguments come back as -1 with a message and nothing is launched (so this
    runs without a GPU)."""
    import qfm
    lib = qfm.load()
    lib.qfm_init(C.byref(qfm.QfmConfig(2048, 512, 512, 10, 1, 1)))
    calls = {
        "qf_rtr_gemv_launch_ex": (None, None, None, None),
        "qf_rtr_topk10_launch_ex": (None, None, None, None),
        "qf_rtr_topk10_rows_launch_ex": (None, None, None, 0, None),
        "qf8_i8_gateup_m1_ex": (None, None, None, None, None, None, 10, 1, None),
        "qf8_i8_down_m1_ex": (None, None, None, None, None, None, None, 10, None),
        "qf8_i8_x8_ex": (None, None, None, 30, None),
        "qf8_i8_csr_build_ex": (None, None, 0, None, None, None, None, None, None),
        "qf8_i8_experts_chunk_ex": (None,) * 11 + (0, 0, None, None, 0, None, None),
        "qf5_nvfp4_moe_all_ex": (None,) * 15 + (0, None),
        "qf5_nvfp4_gateup_all_launch_ex": (None,) * 10 + (0, None),
        "qf5_nvfp4_downacc_all_launch_ex": (None,) * 8 + (0, None),
        "qf5_m8_gateup_ex": (None,) * 8 + (None, None),
        "qf5_m8_downacc_ex": (None,) * 5 + (None, None),
        "qf5_m8_build_csr_ex": (None, None, 0, 0, 0, 0, 0, None, None, None, None, None, None),
        "qf5_m8_reduce4_ex": (None, None, None, None, None, 8, None),
        "qf8_i8_shexp_m1_ex": (None,) * 4 + (None,) * 9 + (None,),
        "qf_rtr_dispatch_launch_ex": (None,) * 7 + (1, 16, None),
        "qf_rtr_hist_launch_ex": (None, None, None),
        "qf8_fp8_build_desc_ex": (None, None, 1, 10, 0, None, None, None),
        "qf8_fp8_gateup_ex": (None,) * 9,
        "qf8_fp8_downacc_ex": (None,) * 7,
        "qf8_i8_gemv_multi_ex": (None, None, None, None),
        "qf8_i8_hc_m1_ex": (None,) * 19,
        "qfm_hc_wait_timeouts": (None,),
        "qf8_stream_inject_ex": (None, None, None, None),
    }
    for name, args in calls.items():
        rc = getattr(lib, name)(*args)
        assert rc == -1, (name, rc)
        assert lib.qfm_last_error() != b"", name
    # the void forms latch the same error
    lib.qf8_i8_x8(None, None, None, 30, None)
    assert lib.qfm_status() == -1
    assert b"multiple of 32" in lib.qfm_last_error()


def test_gated_shared_expert_needs_gate_vector_on_every_path(built):
    """A gated shared expert without sh_gate_inp is rejected for decode rows and
    for prefill alike (checked before any launch: no GPU needed)."""
    import qfm
    lib = qfm.load()
    lib.qfm_init(C.byref(qfm.QfmConfig(2048, 512, 512, 10, 1, 1)))
    arena = qfm.Qf4ExpCache()
    for f in ("i8_gate", "i8_up", "i8_down", "i8s_gate", "i8s_up", "i8s_down"):
        setattr(arena, f, 0x1000)
    arena.slots, arena.fully_resident = 512, 1
    lay = qfm.QfmLayer()
    lay.arena = C.pointer(arena)
    lay.fmt = qfm.QFM_FMT_INT8
    lay.router = 0x2000
    lay.sh_gate = qfm.Qf8I8Mat(0x3000, 0x3100, 512, 2048)
    lay.sh_up = qfm.Qf8I8Mat(0x4000, 0x4100, 512, 2048)
    lay.sh_down = qfm.Qf8I8Mat(0x5000, 0x5100, 2048, 512)
    lay.sh_gate_inp = None
    for M in (1, 8, 9, 300):
        wsb = lib.qfm_workspace_bytes(M)
        rc = lib.qfm_moe_forward(C.byref(lay), 0x6000, M, 0x7000, 0x100000, wsb, None)
        assert rc == -1, (M, rc)
        assert b"sh_gate_inp" in lib.qfm_last_error(), M


def test_fused_forward_needs_a_fully_resident_arena(built):
    """The fused forward addresses expert e at slot e: a partly resident cache
    or an NVFP4 staging ring is rejected before any launch."""
    import qfm
    lib = qfm.load()
    lib.qfm_init(C.byref(qfm.QfmConfig(2048, 512, 512, 10, 1, 0)))
    arena = qfm.Qf4ExpCache()
    for f in ("i8_gate", "i8_up", "i8_down", "i8s_gate", "i8s_up", "i8s_down", "w_gate", "w_up", "w_down",
              "s_gate", "s_up", "s_down", "s2g_dev", "s2u_dev", "s2d_dev"):
        setattr(arena, f, 0x1000)
    lay = qfm.QfmLayer()
    lay.arena = C.pointer(arena)
    lay.router = 0x2000
    wsb = lib.qfm_workspace_bytes(1)
    for slots, resident, ring, fmt in ((192, 0, 0, qfm.QFM_FMT_INT8), (512, 0, 0, qfm.QFM_FMT_INT8),
                                       (512, 1, 2, qfm.QFM_FMT_NVFP4)):
        arena.slots, arena.fully_resident, arena.nv_ring = slots, resident, ring
        lay.fmt = fmt
        lib.qfm_last_error()
        assert lib.qfm_moe_forward(C.byref(lay), 0x6000, 1, 0x7000, 0x100000, wsb, None) == -1
        assert lib.qfm_last_error()
    lib.qfm_init(C.byref(qfm.QfmConfig(2048, 512, 512, 10, 1, 1)))
