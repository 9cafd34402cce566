"""ctypes loader for libobjeta_hip.so (the C ABI declared in include/objeta_hip.h).

The library is built in-tree by __graft_entry__.build() (objeta_amd/csrc/Makefile)
into objeta_amd/lib/. Loading fails loudly when it is missing: there is no CPU
fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libobjeta_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "objeta_hip.h")

_lib = None

P = C.c_void_p
I32 = C.c_int32
U32 = C.c_uint32
U64 = C.c_uint64
I64 = C.c_int64
F32 = C.c_float


class Error(C.Structure):
    _fields_ = [("kind", I32), ("line", U32), ("action", C.c_char * 160), ("file", C.c_char * 96),
                ("module", C.c_char * 64), ("source_message", C.c_char * 320)]


class InitOptions(C.Structure):
    _fields_ = [("device_ordinal", U64), ("stream_count", U64)]


class DeviceInfo(C.Structure):
    _fields_ = [("ordinal", U64), ("name", C.c_char * 256), ("arch", C.c_char * 64),
                ("total_global_mem_bytes", U64), ("compute_capability_major", I32),
                ("compute_capability_minor", I32), ("driver_version", I32), ("runtime_version", I32),
                ("compute_units", I32), ("wavefront_size", I32), ("l2_cache_bytes", I32),
                ("max_shared_memory_per_block", I32), ("clock_khz", I32), ("memory_clock_khz", I32),
                ("memory_bus_width_bits", I32), ("reserved", I32)]


class ExpertPtrs(C.Structure):
    _fields_ = [("gate", P), ("up", P), ("down", P), ("gate_scale", P), ("up_scale", P),
                ("down_scale", P)]


class CacheKey(C.Structure):
    _fields_ = [("layer_id", U64), ("expert_id", U64), ("tensor_kind", I32), ("quant_format", I32)]


class CacheStats(C.Structure):
    _fields_ = [(n, U64) for n in (
        "capacity_bytes", "resident_bytes", "pinned_bytes", "hit_count", "miss_count", "eviction_count",
        "cache_insert_attempt_count", "cache_insert_accept_count", "cache_insert_bypass_count",
        "oversized_tensor_bypass_count", "oversized_expert_bypass_count", "self_eviction_risk_count",
        "entry_count", "device_bytes_reserved")] + [("bypass_oversized_experts", I32), ("reserved", I32)]


class HostExpert(C.Structure):
    _fields_ = [("gate", P), ("gate_len", U64), ("up", P), ("up_len", U64), ("down", P), ("down_len", U64),
                ("gate_scale", P), ("gate_scale_len", U64), ("up_scale", P), ("up_scale_len", U64),
                ("down_scale", P), ("down_scale_len", U64)]


_TEL_U64_HEAD = ("selected_expert_count", "logical_expert_bytes_requested", "actual_expert_bytes_loaded",
                 "resident_cache_bytes_reused", "weight_bytes_loaded", "weight_bytes_reused",
                 "scale_bytes_loaded", "scale_bytes_reused", "resident_cache_resident_bytes",
                 "resident_cache_capacity_bytes", "resident_cache_hit_count", "resident_cache_miss_count",
                 "resident_cache_eviction_count", "resident_cache_insert_attempt_count",
                 "resident_cache_insert_accept_count", "resident_cache_insert_bypass_count",
                 "resident_cache_oversized_tensor_bypass_count",
                 "resident_cache_oversized_expert_bypass_count", "resident_cache_self_eviction_risk_count",
                 "dequantized_scratch_bytes")
_TEL_F32 = ("h2d_ms", "gate_up_qgemv_ms", "activation_ms", "down_qgemv_ms", "accum_ms", "unaccounted_ms",
            "total_ms", "shared_expert_ms")
_TEL_U64_TAIL = ("bytes_by_tensor_kind_gate", "bytes_by_tensor_kind_up", "bytes_by_tensor_kind_down",
                 "bytes_per_expert", "selected_working_set_bytes", "routed_fp4_bytes_loaded",
                 "routed_fp4_bytes_reused", "shared_fp8_bytes_loaded", "shared_fp8_bytes_reused",
                 "total_logical_bytes", "total_loaded_bytes", "total_reused_bytes")


class MoeTelemetry(C.Structure):
    _fields_ = ([(n, U64) for n in _TEL_U64_HEAD] + [(n, F32) for n in _TEL_F32] +
                [(n, U64) for n in _TEL_U64_TAIL])


class CachedLayer(C.Structure):
    _fields_ = [("experts", P), ("n_experts", U64), ("d_router_w", P), ("d_router_bias", P), ("layer_id", U64)]


class StackTelemetry(C.Structure):
    _fields_ = [(n, U64) for n in (
        "layers", "tokens", "logical_expert_bytes_requested", "actual_expert_bytes_loaded",
        "resident_cache_bytes_reused", "distinct_experts", "prefetch_experts_predicted", "prefetch_experts_correct",
        "prefetch_tensors_issued", "prefetch_bytes_issued")] + [(n, F32) for n in (
        "total_ms", "copy_ms", "host_wait_ms", "reserved")]


class QGemvTelemetry(C.Structure):
    _fields_ = [("h2d_ms", F32), ("kernel_ms", F32), ("d2h_ms", F32), ("unaccounted_ms", F32),
                ("total_ms", F32), ("effective_gbps", F32), ("bytes_read", U64)]


# name -> (restype, argtypes)
SIGNATURES = {
    "objeta_hip_last_error": (I32, [P]),
    "objeta_hip_clear_error": (None, []),
    "objeta_hip_abi_version": (I32, []),
    "objeta_hip_block_size": (I32, [I32]),
    "objeta_hip_block_bytes": (I32, [I32]),
    "objeta_hip_quantized_matrix_bytes": (I64, [I32, U64, U64]),
    "objeta_hip_device_count": (I32, [P]),
    "objeta_hip_discover_device": (I32, [U64, P]),
    "objeta_hip_init": (I32, [P, P]),
    "objeta_hip_destroy": (I32, [P]),
    "objeta_hip_device_info_get": (I32, [P, P]),
    "objeta_hip_stream_get": (I32, [P, U64, P]),
    "objeta_hip_stream_synchronize": (I32, [P, P]),
    "objeta_hip_malloc": (I32, [P, U64, P]),
    "objeta_hip_free": (I32, [P, P]),
    "objeta_hip_alloc_pinned_host": (I32, [P, U64, P]),
    "objeta_hip_free_pinned_host": (I32, [P, P]),
    "objeta_hip_copy_h2d": (I32, [P, P, P, P, U64]),
    "objeta_hip_copy_d2h": (I32, [P, P, P, P, U64]),
    "objeta_hip_copy_d2d": (I32, [P, P, P, P, U64]),
    "objeta_hip_zero_device": (I32, [P, P, P, U64]),
    "objeta_hip_event_create": (I32, [P, P]),
    "objeta_hip_event_record": (I32, [P, P, P]),
    "objeta_hip_event_elapsed_ms": (I32, [P, P, P, P]),
    "objeta_hip_event_destroy": (I32, [P, P]),
    "objeta_hip_graph_begin_capture": (I32, [P, P]),
    "objeta_hip_graph_end_capture": (I32, [P, P, P]),
    "objeta_hip_graph_launch": (I32, [P, P, P]),
    "objeta_hip_graph_destroy": (I32, [P, P]),
    "objeta_hip_qgemv": (I32, [P, I32, P, P, U64, P, U64, U64, U64, P, P]),
    "objeta_hip_qgemv_device": (I32, [P, I32, P, P, P, P, U64, U64, U64]),
    "objeta_hip_fp4_gemv_split_device": (I32, [P, P, P, P, P, P, U64, U64, U64]),
    "objeta_hip_quantize_matrix_device": (I32, [P, I32, P, P, U64, U64, P]),
    "objeta_hip_fill_gauss_device": (I32, [P, P, P, U64, U64, U64, F32]),
    "objeta_hip_fill_gauss_quantized_device": (I32, [P, I32, P, P, U64, U64, U64, F32]),
    "objeta_hip_fp4_scale_raw_host": (I32, [P, P, U64]),
    "objeta_hip_fill_fp4_split_device": (I32, [P, P, P, P, U64, U64, U64]),
    "objeta_hip_router_topk_device": (I32, [P, P, P, P, P, U64, U64, U64, U64, I32, P, P]),
    "objeta_hip_router_softmax_exp_device": (I32, [P, P, P, P, U64]),
    "objeta_hip_moe_selected_device": (I32, [P, I32, P, P, U64, P, P, U64, U64, P, P, P, U64, U64,
                                             U64, F32]),
    "objeta_hip_moe_selected_device_noalloc": (I32, [P, I32, P, P, U64, P, P, U64, U64, P, P, P, U64, U64,
                                                     U64, F32]),
    "objeta_hip_moe_selected_shared_device": (I32, [P, I32, P, P, U64, P, P, P, U64, U64, P, P, P, U64, U64,
                                                    U64, F32]),
    "objeta_hip_moe_layer_shared_device": (I32, [P, I32, P, P, U64, P, P, P, U64, I32, U64, P, P, P, P, P,
                                                 U64, U64, U64, F32]),
    "objeta_hip_moe_layer_device": (I32, [P, I32, P, P, U64, P, P, U64, I32, U64, P, P, P, P, P,
                                          U64, U64, U64, F32]),
    "objeta_hip_device_error": (I32, [P, P]),
    "objeta_hip_moe_grouped_device": (I32, [P, I32, P, P, U64, P, P, U64, U64, P, P, P, U64, U64, U64, F32]),
    "objeta_hip_moe_gate_up_device": (I32, [P, I32, P, P, U64, P, U64, U64, P, P, U64, U64, F32]),
    "objeta_hip_moe_down_device": (I32, [P, I32, P, P, U64, P, P, U64, U64, P, P, P, U64, U64]),
    "objeta_hip_cache_create": (I32, [P, U64, P]),
    "objeta_hip_cache_destroy": (I32, [P]),
    "objeta_hip_cache_stats_get": (I32, [P, P]),
    "objeta_hip_cache_set_bypass_oversized_experts": (I32, [P, I32]),
    "objeta_hip_cache_get": (I32, [P, P, P, P, P]),
    "objeta_hip_cache_insert": (I32, [P, P, P, U64, P, P, P]),
    "objeta_hip_cache_get_or_insert": (I32, [P, P, P, U64, P, P, P, P]),
    "objeta_hip_cache_insert_pinned": (I32, [P, P, P, U64, P, P]),
    "objeta_hip_cache_pin": (I32, [P, P]),
    "objeta_hip_cache_touch": (I32, [P, P]),
    "objeta_hip_cache_evict_lru": (I32, [P, P, P]),
    "objeta_hip_cache_clear": (I32, [P]),
    "objeta_hip_cache_reset_counters": (I32, [P]),
    "objeta_hip_cache_release_transient": (I32, [P, P]),
    "objeta_hip_cache_order": (I32, [P, P, U64, P]),
    "objeta_hip_moe_execute_selected": (I32, [P, I32, P, P, U64, P, P, U64, P, U64, U64, U64, U64, U64, P,
                                              P, P]),
    "objeta_hip_act_quant_fp8_device": (I32, [P, P, P, U64, U64, P, P, P]),
    "objeta_hip_fp8_act_fp4_weight_gemv_device": (I32, [P, P, P, P, P, P, P, U64, U64, U64]),
    "objeta_hip_fp8_act_fp8_weight_gemv_device": (I32, [P, P, P, P, P, P, P, U64, U64, U64]),
    "objeta_hip_moe_official_fp4_device": (I32, [P, P, P, U64, P, P, P, U64, U64, P, P, U64, U64, U64, F32,
                                                 P, P]),
    "objeta_hip_moe_execute_official_fp4": (I32, [P, P, P, U64, P, P, U64, P, U64, U64, U64, U64, U64, P, P,
                                                  I32, F32, P, P]),
    "objeta_hip_cache_prefetch": (I32, [P, P, P, P, U64, P]),
    "objeta_hip_moe_stack_cached": (I32, [P, I32, P, P, U64, U64, I32, U64, P, U64, U64, P, I32, P, P, P, P]),
    "objeta_hip_cache_preload_shared": (I32, [P, P, U64, U64, P, P, P]),
    "objeta_hip_st_open": (I32, [C.c_char_p, P]),
    "objeta_hip_st_close": (I32, [P]),
    "objeta_hip_st_len": (I32, [P, P]),
    "objeta_hip_st_key": (I32, [P, U64, P, U64, P]),
    "objeta_hip_st_info_get": (I32, [P, C.c_char_p, P, P]),
    "objeta_hip_st_get_raw": (I32, [P, C.c_char_p, P, P]),
    "objeta_hip_st_get_f32": (I32, [P, C.c_char_p, P, U64, P]),
    "objeta_hip_st_deepseek_expert": (I32, [P, U64, U64, I32, P, P, P, P]),
    "objeta_hip_st_deepseek_shared_expert": (I32, [P, U64, I32, P, P, P, P]),
    "objeta_hip_st_deepseek_router": (I32, [P, U64, I32, P, U64, P]),
}


class LibraryMissing(RuntimeError):
    pass


def header_functions(path: str = HEADER) -> list:
    """Names of every function declared in include/objeta_hip.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(objeta_hip_[a-z0-9_]+)\s*\(", text)))


def load():
    """Load libobjeta_hip.so (raises LibraryMissing if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
