"""ctypes binding of libqfm.so (the C ABI declared in include/qf_moe.h).

This is the Python side of the boundary used by the tests, the smoke check
and bench.py: it loads the in-tree HIP library, mirrors its structs and
declares every exported entry point. It computes nothing itself. Loading
fails loudly when the library has not been built; there is no fallback.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqfm.so")

QFM_FMT_INT8 = 0
QFM_FMT_NVFP4 = 1
GEN_I8, GEN_ROWSCALE, GEN_GAUSS_F32, GEN_GAUSS_BF16, GEN_FP4BYTE, GEN_E4M3SCALE = range(6)

vp = C.c_void_p


class QfmConfig(C.Structure):
    _fields_ = [("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int),
                ("top_k", C.c_int), ("renorm", C.c_int), ("shared_gated", C.c_int)]


class Qf4ExpCache(C.Structure):
    """Byte-compatible with the reference's Qf4ExpCache (qf_nvfp4_wave64.h:133-173)."""
    _fields_ = [("layer", C.c_int), ("slots", C.c_int),
                ("w_gate", vp), ("w_up", vp), ("w_down", vp),
                ("w8_gate", vp), ("w8_up", vp), ("w8_down", vp),
                ("sc_gate", vp), ("sc_up", vp), ("sc_down", vp),
                ("i8_gate", vp), ("i8_up", vp), ("i8_down", vp),
                ("i8s_gate", vp), ("i8s_up", vp), ("i8s_down", vp),
                ("nv_ring", C.c_int),
                ("s_gate", vp), ("s_up", vp), ("s_down", vp),
                ("slot_for_expert", vp), ("expert_in_slot", vp), ("age", vp), ("clock", C.c_uint64),
                ("s2g", vp), ("s2u", vp), ("s2d", vp),
                ("fully_resident", C.c_int),
                ("slot_for_expert_dev", vp), ("expert_in_slot_dev", vp), ("age_dev", vp), ("clock_dev", vp),
                ("s2g_dev", vp), ("s2u_dev", vp), ("s2d_dev", vp),
                ("route_slot_dev", vp), ("mb_host", vp), ("mb_dev", vp),
                ("expected_seq", C.c_uint32)]


class Qf8I8Mat(C.Structure):
    _fields_ = [("w", vp), ("s", vp), ("rows", C.c_int), ("K", C.c_int)]


class Qf5M8Route(C.Structure):
    _fields_ = [("n_exp", C.c_int), ("n_pairs", C.c_int), ("M", C.c_int), ("n_exp_max", C.c_int),
                ("n_exp_dev", vp), ("exp_slot", vp), ("exp_ptr", vp), ("pair_tok", vp), ("pair_wt", vp)]


class QfmLayer(C.Structure):
    _fields_ = [("arena", C.POINTER(Qf4ExpCache)), ("fmt", C.c_int),
                ("router", vp), ("router_bias", vp),
                ("sh_gate", Qf8I8Mat), ("sh_up", Qf8I8Mat), ("sh_down", Qf8I8Mat),
                ("sh_gate_inp", vp)]


class QfmSynthLayer(C.Structure):
    _fields_ = [("layer", QfmLayer), ("arena", Qf4ExpCache)]


class QfRec(C.Structure):
    """Byte-compatible with the reference's QfRec (ocho/amd_server/qwenflash.h:12-24)."""
    _fields_ = [("file_idx", C.c_uint32), ("dtype", C.c_uint32), ("ne", C.c_uint64 * 4),
                ("data_off", C.c_uint64), ("nbytes", C.c_uint64), ("scale2_off", C.c_uint64),
                ("input_off", C.c_uint64), ("scale2_file", C.c_uint32), ("input_file", C.c_uint32),
                ("flags", C.c_uint32)]


class QfEntry(C.Structure):
    """One 512-byte manifest record (qwenflash.h:26-30)."""
    _fields_ = [("name", C.c_char * 256), ("rec", QfRec), ("_pad", C.c_uint8 * 168)]


class QfStore(C.Structure):
    """The opened store (qwenflash.h:32-39)."""
    _fields_ = [("n_shards", C.c_int), ("shard_paths", vp), ("shard_fds", C.POINTER(C.c_int)),
                ("shard_maps", C.POINTER(vp)), ("shard_sizes", C.POINTER(C.c_size_t)),
                ("entries", C.POINTER(QfEntry)), ("n_entries", C.c_int)]


class Qf4ExpXfer(C.Structure):
    """Per-GPU transfer context (qf_nvfp4_wave64.h:178-183)."""
    _fields_ = [("buf", vp * 2), ("ev", vp * 2), ("cur", C.c_int), ("xfer", vp)]


class QfRouteMailbox(C.Structure):
    """Miss mailbox (qwenflash.h:73-83)."""
    _fields_ = [("seq", C.c_uint32), ("miss_n", C.c_uint32), ("miss_expert", C.c_int32 * 16),
                ("miss_slot", C.c_int32 * 16)]


class Qf8I8Multi(C.Structure):
    """Up to 4 INT8 matrices sharing one X8 row (qf8_dense_i8.h:31-32)."""
    _fields_ = [("m", C.POINTER(Qf8I8Mat) * 4), ("y", vp * 4), ("act", C.c_int * 4), ("n", C.c_int)]


class Qf8ShexpW(C.Structure):
    """bf16 shared-expert weights (qf8_dense.h:275-277)."""
    _fields_ = [("gate", vp), ("up", vp), ("down", vp), ("gate_inp", vp)]


class Qf8MoeDesc(C.Structure):
    """FP8 path expert descriptor (qf8_moe_fp8.h:37-44)."""
    _fields_ = [("slot", C.c_int), ("nrow", C.c_int), ("row", C.c_int * 16), ("wt", C.c_float * 16)]


DTYPE_CODES = {"BF16": 1, "F32": 2, "U8": 3, "F8_E4M3": 4, "I64": 5, "F16": 6, "I8": 7, "I32": 8,
               "F64": 9, "F8_E5M2": 10, "I16": 11, "U16": 12, "U32": 13, "U64": 14, "BOOL": 15}
EXPCACHE_NVFP4, EXPCACHE_INT8, EXPCACHE_INT8_ONLY, EXPCACHE_FP8 = 1, 2, 4, 8


class QfmWsView(C.Structure):
    _fields_ = [("logits", vp), ("sel", vp), ("wts", vp), ("hidden", vp), ("counters", vp)]


# name -> (restype, argtypes)
_SIGS = {
    "qfm_init": (C.c_int, [C.POINTER(QfmConfig)]),
    "qfm_get_config": (C.c_int, [C.POINTER(QfmConfig)]),
    "qfm_last_error": (C.c_char_p, []),
    "qfm_status": (C.c_int, []),
    "qfm_version": (C.c_char_p, []),
    "qfm_set_hbm_budget": (C.c_int, [C.c_size_t]),
    "qfm_get_hbm_budget": (C.c_size_t, []),
    "qfm_arena_bytes": (C.c_size_t, [C.c_int]),
    "qfm_expcache_bytes": (C.c_size_t, [C.c_int, C.c_int]),
    "qfm_sizeof": (C.c_size_t, [C.c_int]),
    "qf_rtr_gemv_launch": (None, [vp, vp, vp, vp]),
    "qf_rtr_topk10_launch": (None, [vp, vp, vp, vp]),
    "qf_rtr_topk10_rows_launch": (None, [vp, vp, vp, C.c_int, vp]),
    "qfm_router_logits": (C.c_int, [vp, vp, vp, C.c_int, vp, vp]),
    "qfm_topk": (C.c_int, [vp, C.c_int, vp, vp, vp]),
    "qf8_i8_gateup_m1": (None, [C.POINTER(Qf4ExpCache), vp, vp, vp, vp, vp, C.c_int, C.c_int, vp]),
    "qf8_i8_down_m1": (None, [C.POINTER(Qf4ExpCache), vp, vp, vp, vp, vp, vp, C.c_int, vp]),
    "qf8_i8_x8": (None, [vp, vp, vp, C.c_int, vp]),
    "qf8_i8_csr_build": (None, [vp, vp, C.c_int, vp, vp, vp, vp, vp, vp]),
    "qf8_i8_experts_chunk": (None, [C.POINTER(Qf4ExpCache), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, C.c_int,
                                    C.c_int, vp, vp, C.c_int, vp, vp]),
    "qf8_i8_build": (C.c_int, [C.POINTER(Qf4ExpCache), vp]),
    "qf8_i8_build_slot": (C.c_int, [C.POINTER(Qf4ExpCache), C.c_int, C.c_int, C.c_int, vp]),
    "qf5_nvfp4_moe_all": (None, [vp] * 15 + [C.c_int, vp]),
    "qf5_nvfp4_gateup_all_launch": (None, [vp] * 10 + [C.c_int, vp]),
    "qf5_nvfp4_downacc_all_launch": (None, [vp] * 8 + [C.c_int, vp]),
    "qf5_m8_gateup": (None, [vp] * 8 + [C.POINTER(Qf5M8Route), vp]),
    "qf5_m8_downacc": (None, [vp] * 5 + [C.POINTER(Qf5M8Route), vp]),
    "qf5_m8_build_csr": (None, [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, vp, vp, vp, vp]),
    "qf5_m8_reduce4": (None, [vp, vp, vp, vp, vp, C.c_int, vp]),
    "qf8_i8_shexp_m1": (None, [C.POINTER(Qf8I8Mat)] * 4 + [vp] * 9 + [vp]),
    "qf8_i8_shexp_rows": (C.c_int, [C.POINTER(Qf8I8Mat)] * 4 + [vp] * 9 + [C.c_int, vp]),
    "qf_rtr_gemv_launch_ex": (C.c_int, [vp, vp, vp, vp]),
    "qf_rtr_topk10_launch_ex": (C.c_int, [vp, vp, vp, vp]),
    "qf_rtr_topk10_rows_launch_ex": (C.c_int, [vp, vp, vp, C.c_int, vp]),
    "qf8_i8_gateup_m1_ex": (C.c_int, [C.POINTER(Qf4ExpCache), vp, vp, vp, vp, vp, C.c_int, C.c_int, vp]),
    "qf8_i8_down_m1_ex": (C.c_int, [C.POINTER(Qf4ExpCache), vp, vp, vp, vp, vp, vp, C.c_int, vp]),
    "qf8_i8_x8_ex": (C.c_int, [vp, vp, vp, C.c_int, vp]),
    "qf8_i8_csr_build_ex": (C.c_int, [vp, vp, C.c_int, vp, vp, vp, vp, vp, vp]),
    "qf8_i8_experts_chunk_ex": (C.c_int, [C.POINTER(Qf4ExpCache), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                          C.c_int, C.c_int, vp, vp, C.c_int, vp, vp]),
    "qf5_nvfp4_moe_all_ex": (C.c_int, [vp] * 15 + [C.c_int, vp]),
    "qf5_nvfp4_gateup_all_launch_ex": (C.c_int, [vp] * 10 + [C.c_int, vp]),
    "qf5_nvfp4_downacc_all_launch_ex": (C.c_int, [vp] * 8 + [C.c_int, vp]),
    "qf5_m8_gateup_ex": (C.c_int, [vp] * 8 + [C.POINTER(Qf5M8Route), vp]),
    "qf5_m8_downacc_ex": (C.c_int, [vp] * 5 + [C.POINTER(Qf5M8Route), vp]),
    "qf5_m8_build_csr_ex": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, vp, vp, vp, vp]),
    "qf5_m8_reduce4_ex": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, vp]),
    "qf8_i8_shexp_m1_ex": (C.c_int, [C.POINTER(Qf8I8Mat)] * 4 + [vp] * 9 + [vp]),
    "qfm_workspace_bytes": (C.c_size_t, [C.c_int]),
    "qfm_workspace_view": (C.c_int, [vp, C.c_int, C.POINTER(QfmWsView)]),
    "qfm_moe_forward": (C.c_int, [C.POINTER(QfmLayer), vp, C.c_int, vp, vp, C.c_size_t, vp]),
    "qfm_moe_forward_f32": (C.c_int, [C.POINTER(QfmLayer), vp, C.c_int, vp, vp, C.c_size_t, vp]),
    "qfm_moe_forward_noalloc": (C.c_int, [C.POINTER(QfmLayer), vp, C.c_int, vp, vp]),
    "qfm_moe_forward_sections": (C.c_int, [C.POINTER(QfmLayer), vp, C.c_int, vp, vp, C.c_size_t, C.c_int, vp]),
    "qfm_moe_forward_layers": (C.c_int, [C.POINTER(QfmLayer), C.c_int, vp, C.c_long, C.c_int, vp, C.c_long,
                                         vp, C.c_size_t, vp]),
    "qfm_profile_enable": (C.c_int, [C.c_int]),
    "qfm_profile_read": (C.c_int, [C.POINTER(C.c_double), C.c_int, C.POINTER(C.c_int)]),
    "qfm_graph_capture_begin": (C.c_int, [vp]),
    "qfm_graph_capture_end": (vp, [vp]),
    "qfm_graph_launch": (C.c_int, [vp, vp]),
    "qfm_graph_destroy": (C.c_int, [vp]),
    "qfm_gen_fill": (C.c_int, [vp, C.c_int, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32,
                               C.c_float, vp]),
    "qfm_fill_f32": (C.c_int, [vp, C.c_uint64, C.c_float, vp]),
    "qfm_arena_init": (C.c_int, [C.POINTER(Qf4ExpCache), C.c_int, C.c_int]),
    "qfm_arena_generate": (C.c_int, [C.POINTER(Qf4ExpCache), C.c_uint32, C.c_uint32, vp]),
    "qfm_arena_free": (None, [C.POINTER(Qf4ExpCache)]),
    "qfm_synth_layer_create": (C.c_int, [C.POINTER(QfmSynthLayer), C.c_int, C.c_uint32, C.c_uint32, C.c_int, vp]),
    "qfm_synth_layer_destroy": (None, [C.POINTER(QfmSynthLayer)]),
    "qf_store_open": (C.c_int, [C.POINTER(QfStore), C.c_char_p]),
    "qf_find": (C.POINTER(QfEntry), [C.POINTER(QfStore), C.c_char_p]),
    "qf_store_close": (None, [C.POINTER(QfStore)]),
    "qfm_store_data": (vp, [C.POINTER(QfStore), C.POINTER(QfEntry)]),
    "qf4_expxfer_init": (C.c_int, [C.POINTER(Qf4ExpXfer)]),
    "qf4_expxfer_free": (None, [C.POINTER(Qf4ExpXfer)]),
    "qf4_expcache_init": (C.c_int, [C.POINTER(Qf4ExpCache), C.POINTER(QfStore), C.c_int, C.c_int]),
    "qfm_expcache_init": (C.c_int, [C.POINTER(Qf4ExpCache), C.POINTER(QfStore), C.c_int, C.c_int, C.c_int]),
    "qf4_expcache_free": (None, [C.POINTER(Qf4ExpCache)]),
    "qf4_expcache_prefill": (C.c_int, [C.POINTER(Qf4ExpCache), C.POINTER(QfStore), C.POINTER(Qf4ExpXfer), vp]),
    "qf4_expcache_prepare": (C.c_int, [C.POINTER(Qf4ExpCache), C.POINTER(QfStore), C.POINTER(Qf4ExpXfer),
                                       C.c_int, vp]),
    "qf4_expcache_service": (C.c_int, [C.POINTER(Qf4ExpCache), C.POINTER(QfStore), C.POINTER(Qf4ExpXfer), vp]),
    "qf4_expcache_stats": (None, [C.POINTER(C.c_ulonglong)] * 3),
    "qf8_fp8_pack_expert": (C.c_int, [vp, vp, C.c_float, C.c_int, C.c_int, vp, vp]),
    "qf8_i8_quant_bf16": (C.c_int, [vp, C.c_int, C.c_int, C.POINTER(Qf8I8Mat), vp]),
    "qf8_i8_quant_bf16_host": (C.c_int, [vp, C.c_int, C.c_int, C.POINTER(Qf8I8Mat), vp]),
    "qfm_layer_load": (C.c_int, [C.POINTER(QfmSynthLayer), C.POINTER(QfStore), C.c_int, C.c_int,
                                 C.POINTER(Qf4ExpXfer), vp]),
    "qfm_store_check_layer": (C.c_int, [C.POINTER(QfStore), C.c_int]),
    "qf_rtr_dispatch_launch": (None, [vp] * 7 + [C.c_uint32, C.c_int, vp]),
    "qf_rtr_dispatch_launch_ex": (C.c_int, [vp] * 7 + [C.c_uint32, C.c_int, vp]),
    "qf_rtr_hist_launch": (None, [vp, vp, vp]),
    "qf_rtr_hist_launch_ex": (C.c_int, [vp, vp, vp]),
    "qf8_fp8_build_desc": (None, [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp, vp]),
    "qf8_fp8_build_desc_ex": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp, vp]),
    "qf8_fp8_gateup": (None, [vp] * 9),
    "qf8_fp8_gateup_ex": (C.c_int, [vp] * 9),
    "qf8_fp8_downacc": (None, [vp] * 7),
    "qf8_fp8_downacc_ex": (C.c_int, [vp] * 7),
    "qf8_i8_gemv_multi": (None, [C.POINTER(Qf8I8Multi), vp, vp, vp]),
    "qf8_i8_gemv_multi_ex": (C.c_int, [C.POINTER(Qf8I8Multi), vp, vp, vp]),
    "qf8_i8_gemv_rows": (C.c_int, [C.POINTER(Qf8I8Multi), vp, vp, C.c_int, vp]),
    "qf8_i8_hc_m1": (None, [vp] * 6 + [C.POINTER(Qf8I8Mat)] * 3 + [vp] * 9 + [vp]),
    "qf8_i8_hc_m1_ex": (C.c_int, [vp] * 6 + [C.POINTER(Qf8I8Mat)] * 3 + [vp] * 9 + [vp]),
    "qf8_i8_hc_rows": (C.c_int, [vp] * 6 + [C.POINTER(Qf8I8Mat)] * 3 + [vp] * 9 + [C.c_int, vp]),
    "qfm_hc_premix": (C.c_int, [vp] * 6 + [C.POINTER(Qf8I8Mat)] * 3 + [vp] * 10 + [C.c_int, vp]),
    "qfm_hc_wait_timeouts": (C.c_int, [C.POINTER(C.c_uint32)]),
    "qf8_stream_inject": (None, [vp, vp, vp, vp]),
    "qf8_stream_inject_ex": (C.c_int, [vp, vp, vp, vp]),
    "qf8_shexp": (None, [C.POINTER(Qf8ShexpW), vp, vp, vp, vp, vp, vp, vp]),
    "qf8_shexp_ex": (C.c_int, [C.POINTER(Qf8ShexpW), vp, vp, vp, vp, vp, vp, vp]),
    "qf8_shexp_M": (None, [C.POINTER(Qf8ShexpW), vp, C.c_int, vp, vp, vp, vp, vp, C.c_int, C.c_int, vp]),
    "qf8_shexp_M_ex": (C.c_int, [C.POINTER(Qf8ShexpW), vp, C.c_int, vp, vp, vp, vp, vp, C.c_int, C.c_int, vp]),
    "qfm_gen_input_rows": (C.c_int, [vp, C.c_int, C.c_uint32, C.c_uint32, C.c_int, vp]),
    "qfm_dev_malloc": (vp, [C.c_size_t]),
    "qfm_dev_free": (C.c_int, [vp]),
    "qfm_memcpy_h2d": (C.c_int, [vp, vp, C.c_size_t]),
    "qfm_memcpy_d2h": (C.c_int, [vp, vp, C.c_size_t]),
    "qfm_memcpy_d2d": (C.c_int, [vp, vp, C.c_size_t]),
    "qfm_memset": (C.c_int, [vp, C.c_int, C.c_size_t]),
    "qfm_stream_create": (vp, []),
    "qfm_stream_destroy": (C.c_int, [vp]),
    "qfm_stream_sync": (C.c_int, [vp]),
    "qfm_device_sync": (C.c_int, []),
    "qfm_event_create": (vp, []),
    "qfm_event_destroy": (C.c_int, [vp]),
    "qfm_event_record": (C.c_int, [vp, vp]),
    "qfm_event_elapsed_ms": (C.c_float, [vp, vp]),
    "qfm_device_info": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_size_t),
                                  C.POINTER(C.c_int), C.POINTER(C.c_int)]),
}

_lib = None


class QfmError(RuntimeError):
    pass


def load(path=LIB_PATH):
    """Load libqfm.so once; raise if it is missing (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise QfmError(f"{path} is not built: run __graft_entry__.build() (make -C qwen-3-ocho_amd)")
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols():
    return sorted(_SIGS)


def check(rc, what="qfm call"):
    lib = load()
    if rc != 0:
        msg = lib.qfm_last_error().decode()
        raise QfmError(f"{what} failed rc={rc}: {msg}")


def status_check(what="qfm"):
    lib = load()
    st = lib.qfm_status()
    if st != 0:
        raise QfmError(f"{what}: {lib.qfm_last_error().decode()}")


def init(hidden=2048, inter=512, n_experts=512, top_k=10, renorm=1, shared_gated=1):
    lib = load()
    cfg = QfmConfig(hidden, inter, n_experts, top_k, renorm, shared_gated)
    check(lib.qfm_init(C.byref(cfg)), "qfm_init")
    return cfg


class DevBuf:
    """Device allocation owned by Python (freed explicitly or at GC)."""

    def __init__(self, nbytes):
        self.lib = load()
        self.nbytes = int(nbytes)
        self.ptr = self.lib.qfm_dev_malloc(self.nbytes)
        if not self.ptr:
            raise QfmError(f"device alloc of {nbytes} bytes failed: {self.lib.qfm_last_error().decode()}")

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(self.lib.qfm_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes), "h2d")

    def download(self, dtype, shape, offset=0):
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(self.lib.qfm_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes), "d2h")
        return out

    def zero(self):
        check(self.lib.qfm_memset(self.ptr, 0, self.nbytes), "memset")

    def free(self):
        if self.ptr:
            self.lib.qfm_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def d2h(ptr, dtype, shape):
    lib = load()
    out = np.empty(shape, dtype=dtype)
    check(lib.qfm_memcpy_d2h(out.ctypes.data, ptr, out.nbytes), "d2h")
    return out


def device_info():
    lib = load()
    name = C.create_string_buffer(64)
    ncu, mem, ma, mi = C.c_int(), C.c_size_t(), C.c_int(), C.c_int()
    check(lib.qfm_device_info(name, 64, C.byref(ncu), C.byref(mem), C.byref(ma), C.byref(mi)), "device_info")
    return {"arch": name.value.decode(), "cus": ncu.value, "mem_bytes": mem.value}


class Stream:
    def __init__(self):
        self.lib = load()
        self.h = self.lib.qfm_stream_create()
        if not self.h:
            raise QfmError("stream create failed")

    def sync(self):
        check(self.lib.qfm_stream_sync(self.h), "stream sync")

    def destroy(self):
        if self.h:
            self.lib.qfm_stream_destroy(self.h)
            self.h = None


class Event:
    def __init__(self):
        self.lib = load()
        self.h = self.lib.qfm_event_create()

    def record(self, stream):
        check(self.lib.qfm_event_record(self.h, stream.h if isinstance(stream, Stream) else stream), "event record")

    def elapsed_ms(self, later):
        return float(self.lib.qfm_event_elapsed_ms(self.h, later.h))


class SynthLayer:
    """A generated layer living on the device (qfm_synth_layer_create)."""

    def __init__(self, fmt, seed, layer, with_bias=False, stream=None):
        self.lib = load()
        self.s = QfmSynthLayer()
        check(self.lib.qfm_synth_layer_create(C.byref(self.s), fmt, seed, layer, int(with_bias),
                                              stream.h if stream else None), "synth layer")

    @property
    def layer(self):
        return self.s.layer

    def destroy(self):
        if self.s.layer.router:
            self.lib.qfm_synth_layer_destroy(C.byref(self.s))

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Store:
    """An opened weight store (qf_store_open): the reference's manifest
    directory, one .safetensors file, or a directory of them."""

    def __init__(self, path):
        self.lib = load()
        self.st = QfStore()
        check(self.lib.qf_store_open(C.byref(self.st), str(path).encode()), f"qf_store_open({path})")

    def find(self, name):
        p = self.lib.qf_find(C.byref(self.st), name.encode())
        return p.contents if p else None

    def names(self):
        return [self.st.entries[i].name.decode() for i in range(self.st.n_entries)]

    def data(self, entry):
        """The entry's bytes (a copy out of the mapping)."""
        ptr = self.lib.qfm_store_data(C.byref(self.st), C.byref(entry))
        return C.string_at(ptr, entry.rec.nbytes) if entry.rec.nbytes else b""

    def close(self):
        if self.st.entries or self.st.n_shards:
            self.lib.qf_store_close(C.byref(self.st))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ExpXfer:
    """Pinned double-buffered transfer context (qf4_expxfer_init)."""

    def __init__(self):
        self.lib = load()
        self.x = Qf4ExpXfer()
        check(self.lib.qf4_expxfer_init(C.byref(self.x)), "qf4_expxfer_init")

    def free(self):
        if self.x.xfer:
            self.lib.qf4_expxfer_free(C.byref(self.x))

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class LoadedLayer(SynthLayer):
    """A MoE layer read from a weight store (qfm_layer_load)."""

    def __init__(self, store, layer, fmt, xfer, stream=None):
        self.lib = load()
        self.s = QfmSynthLayer()
        check(self.lib.qfm_layer_load(C.byref(self.s), C.byref(store.st), layer, fmt, C.byref(xfer.x),
                                      stream.h if stream else None), f"qfm_layer_load(layer {layer})")
