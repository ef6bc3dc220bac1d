"""Loading and declaring libnaiwa_moe.so (the gfx950 C ABI of include/naiwa_moe.h).

The product path has no fallback: if the shared library is missing or fails to
load, every entry point raises.  Build it with ``python naiwa-rs_amd/build.py``
(or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes as C
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# NAIWA_MOE_LIB: load another build of the same ABI (e.g. an alternative kernel build)
LIB_PATH = os.environ.get("NAIWA_MOE_LIB") or os.path.join(PKG_ROOT, "libnaiwa_moe.so")

OK = 0
E_INVALID, E_UNSUPPORTED, E_TIMEOUT, E_NOMEM, E_BAD_ID, E_NOT_FOUND, E_DEVICE = -1, -2, -3, -4, -5, -6, -7
E_FORMAT, E_IO, E_TOO_LARGE = -8, -9, -10

F32, F16, Q8_0, Q4_K, BF16 = 0, 1, 8, 12, 30
ACT_SILU, ACT_GELU_PYTORCH_TANH = 0, 1
ROUTE_SOFTMAX_TOPK_RENORM, ROUTE_TOPK_SOFTMAX, ROUTE_SOFTMAX_TOPK = 0, 1, 2


class NaiwaError(RuntimeError):
    def __init__(self, rc: int, what: str):
        self.rc = rc
        msg = lib().naiwa_status_string(rc).decode() if _lib is not None else str(rc)
        super().__init__(f"{what}: {msg} ({rc})")


class Bank(C.Structure):
    """naiwa_bank: one projection's slot bank (include/naiwa_moe.h)."""
    _fields_ = [("base", C.c_void_p), ("slot_stride", C.c_int64), ("slots", C.c_int32),
                ("n", C.c_int32), ("k", C.c_int32), ("dtype", C.c_int32)]


class Layer(C.Structure):
    """naiwa_layer: router + the three banks + the expert->slot table of one layer."""
    _fields_ = [("router", C.c_void_p), ("gate", Bank), ("up", Bank), ("down", Bank),
                ("slot_of_expert", C.c_void_p)]


STACK_LAYERED, STACK_FUSED = 0, 1

STAGING_RING_FIRST = 1 << 30


class CachedLayerDesc(C.Structure):
    """naiwa_cached_layer_desc (include/naiwa_cached.h)."""
    _fields_ = [("router", C.c_void_p), ("router_bias", C.c_void_p), ("gate", Bank), ("up", Bank),
                ("down", Bank), ("host_gate", C.c_void_p), ("host_up", C.c_void_p), ("host_down", C.c_void_p),
                ("num_experts", C.c_int), ("top_k", C.c_int), ("hidden", C.c_int), ("inter", C.c_int),
                ("usable", C.c_int), ("mode", C.c_int), ("act", C.c_int), ("host_expert_stride", C.c_int64)]


class Copy(C.Structure):
    """naiwa_copy (include/naiwa_moe.h)."""
    _fields_ = [("dst", C.c_void_p), ("src", C.c_void_p), ("bytes", C.c_uint64)]


class Pending(C.Structure):
    """naiwa_pending (include/naiwa_doorbell.h)."""
    _fields_ = [("seq", C.c_uint32), ("len", C.c_int), ("chan", C.c_int)]


TASK_FN = C.CFUNCTYPE(None, C.c_void_p)
RESULT_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_float), C.c_int)


class CachedStep(C.Structure):
    """naiwa_cached_step (include/naiwa_cached.h)."""
    _fields_ = [("hits", C.c_int), ("staged", C.c_int), ("staged_experts", C.c_int), ("promoted", C.c_int),
                ("pcie_bytes", C.c_int64), ("preload_waits", C.c_int), ("cpu", C.c_int)]


class HostExperts(C.Structure):
    """naiwa_host_experts (include/naiwa_cached.h)."""
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p), ("gate_stride", C.c_int64),
                ("up_stride", C.c_int64), ("down_stride", C.c_int64), ("gate_dtype", C.c_int),
                ("up_dtype", C.c_int), ("down_dtype", C.c_int), ("num_experts", C.c_int), ("hidden", C.c_int),
                ("inter", C.c_int)]


class StepPlan(C.Structure):
    """naiwa_step_plan (include/naiwa_policy.h)."""
    _fields_ = [("hits", C.c_int), ("staged", C.c_int), ("staged_experts", C.c_int), ("cpu", C.c_int)]


class LookaheadStep(C.Structure):
    """naiwa_lookahead_step (include/naiwa_cached.h)."""
    _fields_ = [("predicted", C.c_int), ("resident", C.c_int), ("loads", C.c_int), ("swaps", C.c_int),
                ("pcie_bytes", C.c_int64)]


class PrefillStreamDesc(C.Structure):
    """naiwa_prefill_stream_desc (include/naiwa_prefill.h)."""
    _fields_ = [("n_layers", C.c_int), ("num_experts", C.c_int), ("hidden", C.c_int), ("inter", C.c_int),
                ("dtype_gate", C.c_int), ("dtype_up", C.c_int), ("dtype_down", C.c_int),
                ("host_gate", C.POINTER(C.c_void_p)), ("host_up", C.POINTER(C.c_void_p)),
                ("host_down", C.POINTER(C.c_void_p)), ("depth", C.c_int)]


class PrefillStreamStats(C.Structure):
    """naiwa_prefill_stream_stats (include/naiwa_prefill.h)."""
    _fields_ = [("uploads", C.c_uint64), ("upload_bytes", C.c_uint64), ("forwards", C.c_uint64)]


STATS_FIELDS = ("hits", "promotions", "misses", "staged", "lookahead_loads", "swaps", "lookahead_dropped",
                "sync_waits", "pcie_misses", "pcie_bytes", "result_stalls")


class CacheStats(C.Structure):
    """naiwa_cache_stats (include/naiwa_policy.h)."""
    _fields_ = [(f, C.c_uint64) for f in STATS_FIELDS]


_lib: C.CDLL | None = None

vp, i32, i64, u32, u64, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_uint64, C.c_float
_P = C.POINTER

# name -> (restype, argtypes).  Every symbol include/naiwa_moe.h declares is listed.
SIGNATURES: dict[str, tuple] = {
    "naiwa_status_string": (C.c_char_p, [i32]),
    "naiwa_device_count": (i32, [_P(i32)]),
    "naiwa_mem_info": (i32, [_P(u64), _P(u64)]),
    "naiwa_set_device": (i32, [i32]),
    "naiwa_device_info": (i32, [i32, _P(i32), _P(i32), _P(i64), C.c_char_p, i32]),
    "naiwa_malloc": (i32, [_P(vp), C.c_size_t]),
    "naiwa_free": (i32, [vp]),
    "naiwa_host_alloc": (i32, [_P(vp), C.c_size_t]),
    "naiwa_host_free": (i32, [vp]),
    "naiwa_memcpy_h2d": (i32, [vp, vp, C.c_size_t, i64]),
    "naiwa_memcpy_d2h": (i32, [vp, vp, C.c_size_t, i64]),
    "naiwa_memcpy_d2d": (i32, [vp, vp, C.c_size_t, i64]),
    "naiwa_memset": (i32, [vp, i32, C.c_size_t, i64]),
    "naiwa_stream_create": (i32, [_P(i64)]),
    "naiwa_stream_destroy": (i32, [i64]),
    "naiwa_stream_sync": (i32, [i64]),
    "naiwa_stream_wait_event": (i32, [i64, i64]),
    "naiwa_event_create": (i32, [_P(i64), i32]),
    "naiwa_event_destroy": (i32, [i64]),
    "naiwa_event_record": (i32, [i64, i64]),
    "naiwa_event_sync": (i32, [i64]),
    "naiwa_event_query": (i32, [i64]),
    "naiwa_event_elapsed_ms": (i32, [_P(f32), i64, i64]),
    "naiwa_device_sync": (i32, []),
    "naiwa_last_error": (i32, []),
    "doorbell_poll_serve": (i32, [vp, vp, C.c_uint32, C.c_uint32, i64]),
    "doorbell_poll_wait": (i32, [vp, C.c_uint32, i64]),
    "doorbell_poll_signal": (i32, [vp, C.c_uint32, i64]),
    "doorbell_alloc_mapped": (i32, [_P(vp), C.c_size_t]),
    "doorbell_free_host": (i32, [vp]),
    "doorbell_get_device_ptr": (None, [vp, _P(vp)]),
    "doorbell_ring": (None, [vp, vp, vp, vp, vp, i32, i64]),
    "doorbell_copy_f32": (None, [vp, vp, vp, i32, i64]),
    "doorbell_wait_copy_f32": (None, [vp, u32, vp, i64, vp, vp, i32, i64]),
    "naiwa_doorbell_set_wait_limit_us": (i32, [u64]),
    "naiwa_doorbell_timeouts": (i32, [_P(u32)]),
    "naiwa_host_store_release_u32": (None, [vp, u32]),
    "naiwa_host_load_acquire_u32": (u32, [vp]),
    "naiwa_host_wait_ge": (i32, [vp, u32, i64, i64]),
    "naiwa_projection_bytes": (i64, [i32, i64, i64]),
    "naiwa_moe_decode": (i32, [_P(Bank), _P(Bank), _P(Bank), vp, i32, vp, vp, i32, i32, i32, vp, i64]),
    "naiwa_moe_decode_ex": (i32, [_P(Bank), _P(Bank), _P(Bank), vp, i32, vp, vp, i32, i32, i32, vp, i32, i64]),
    "naiwa_moe_decode_noalloc": (i32, [_P(Bank), _P(Bank), _P(Bank), vp, i32, vp, vp, i32, i32, i32, vp, i32, i64]),
    "naiwa_moe_decode_scratch_bytes": (i64, [i32, i32, i32, i32, i32]),
    "naiwa_router_topk": (i32, [vp, i32, vp, i32, i32, i32, i32, i32, vp, vp, vp, i64]),
    "naiwa_router_topk_biased": (i32, [vp, i32, vp, vp, i32, i32, i32, i32, i32, vp, vp, vp, i64]),
    "naiwa_router_topk_ld": (i32, [vp, i32, vp, vp, i32, i32, i32, i32, i32, vp, vp, i32, vp, i64]),
    "naiwa_moe_prefill": (i32, [_P(Bank), _P(Bank), _P(Bank), vp, vp, vp, i32, i32, i32, vp, i32, i64]),
    "naiwa_moe_gather": (i32, [vp, i32, i32, vp, vp, vp, i64]),
    "naiwa_synth": (i32, [i32, u64, u64, i64, f32, f32, vp, i64]),
    "naiwa_stack_decode": (i32, [_P(Layer), i32, vp, i32, i32, i32, i32, i32, i32, vp, vp, i32, i64]),
    "naiwa_stack_decode_y": (i32, [_P(Layer), i32, vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, i32, i64]),
    "naiwa_stack_set_blocks_per_cu": (i32, [i32]),
    "naiwa_stack_status": (i32, [_P(i32), _P(i32)]),
    "naiwa_residual_add_bf16": (i32, [vp, vp, i64, i64]),
    "naiwa_stack_trace_enable": (i32, [i32]),
    "naiwa_stack_trace_read": (i32, [_P(u64), i32, _P(i32), _P(i32)]),
    "naiwa_upload_expert": (i32, [vp, vp, vp, i64, i64, i64]),
    "naiwa_copy_batch": (i32, [_P(Copy), i32, i64]),
    "naiwa_memcpy_2d_d2d": (i32, [vp, C.c_size_t, vp, C.c_size_t, C.c_size_t, C.c_size_t, i64]),
    "naiwa_memcpy_2d": (i32, [vp, C.c_size_t, vp, C.c_size_t, C.c_size_t, C.c_size_t, i64]),
    # include/naiwa_doorbell.h
    "naiwa_topk_doorbell_create": (i32, [i32, _P(vp)]),
    "naiwa_topk_doorbell_destroy": (i32, [vp]),
    "naiwa_topk_doorbell_publish_and_read": (i32, [vp, vp, vp, i32, i64, vp, vp, i64]),
    "naiwa_act_doorbell_create": (i32, [i32, _P(vp)]),
    "naiwa_act_doorbell_destroy": (i32, [vp]),
    "naiwa_act_doorbell_publish": (i32, [vp, vp, i32, u32, i64]),
    "naiwa_act_doorbell_wait_publish": (i32, [vp, u32, i32, vp, i64, _P(i32)]),
    "naiwa_result_doorbell_create": (i32, [i32, _P(vp)]),
    "naiwa_result_doorbell_destroy": (i32, [vp]),
    "naiwa_result_doorbell_max_n": (i32, [vp]),
    "naiwa_result_doorbell_publish": (i32, [vp, vp, i32, u32, _P(i32)]),
    "naiwa_result_doorbell_wait_copy": (i32, [vp, u32, i32, vp, i64]),
    "naiwa_result_doorbell_consumed": (i32, [vp, _P(u32)]),
    "naiwa_pass_cell_create": (i32, [_P(vp)]),
    "naiwa_pass_cell_destroy": (i32, [vp]),
    "naiwa_pass_cell_claim": (i32, [vp, i64, _P(u32)]),
    "naiwa_pass_cell_wait_latest": (i32, [vp, i64, _P(u32)]),
    "naiwa_pass_cell_claimed": (i32, [vp, _P(u32)]),
    "naiwa_executor_create": (i32, [_P(vp)]),
    "naiwa_executor_destroy": (i32, [vp]),
    "naiwa_executor_submit": (i32, [vp, TASK_FN, vp]),
    "naiwa_executor_is_idle": (i32, [vp]),
    "naiwa_executor_wait_idle": (i32, [vp, i64]),
    "naiwa_executor_submit_result": (i32, [vp, i32, RESULT_FN, vp, _P(Pending)]),
    "naiwa_pending_upload": (i32, [vp, _P(Pending), vp, i64]),
    "naiwa_executor_take_error": (i32, [vp, C.c_char_p, i32]),
    "naiwa_executor_stalls": (i32, [vp, _P(u64)]),
    # include/naiwa_cached.h
    "naiwa_cached_layer_create": (i32, [_P(CachedLayerDesc), vp, i32, i64, _P(vp)]),
    "naiwa_cached_layer_destroy": (i32, [vp]),
    "naiwa_cached_layer_cache": (i32, [vp, _P(vp)]),
    "naiwa_cached_layer_fill": (i32, [vp, i32, _P(i32)]),
    "naiwa_cached_layer_seed": (i32, [vp, vp, i32, f32, _P(i32)]),
    "naiwa_cached_layer_forward": (i32, [vp, vp, i32, vp, f32, i32, u64, i64, _P(CachedStep)]),
    "naiwa_cached_layer_routing": (i32, [vp, vp, vp, i32]),
    "naiwa_cached_layer_forward_ahead": (i32, [vp, vp, i32, vp, i32, vp, f32, i32, u64, i64, _P(CachedStep),
                                               _P(LookaheadStep)]),
    "naiwa_cached_layer_prefetch": (i32, [vp, vp, i32, i32, i64, _P(LookaheadStep)]),
    "naiwa_cached_layer_predicted": (i32, [vp, vp, i32, _P(i32)]),
    "naiwa_cached_layer_set_upload_sync": (i32, [vp, i32]),
    "naiwa_cached_layer_set_upload_path": (i32, [vp, i32]),
    "naiwa_cached_layer_set_cpu_misses": (i32, [vp, i32]),
    "naiwa_cached_layer_upload_timeouts": (i32, [vp, _P(C.c_uint32)]),
    "naiwa_cpu_moe_decode": (i32, [_P(HostExperts), vp, vp, vp, i32, i32, i32, vp]),
    "naiwa_cached_stack_forward": (i32, [vp, i32, vp, i32, vp, f32, i32, u64, i32, i64, _P(CachedStep),
                                         _P(LookaheadStep)]),
    # include/naiwa_policy.h (host only)
    "naiwa_cache_create": (i32, [i32, i32, i32, _P(vp)]),
    "naiwa_cache_destroy": (i32, [vp]),
    "naiwa_cache_route": (i32, [vp, vp, i32, i32, vp]),
    "naiwa_cache_fill_candidate": (i32, [vp, _P(i32), _P(i32)]),
    "naiwa_cache_lru_victim": (i32, [vp, vp, i32, _P(i32), _P(i32), _P(i32)]),
    "naiwa_cache_admit": (i32, [vp, i32, _P(i32)]),
    "naiwa_cache_replace": (i32, [vp, i32, vp, i32, _P(i32)]),
    "naiwa_cache_publish": (i32, [vp, i32]),
    "naiwa_cache_unreserve": (i32, [vp, i32]),
    "naiwa_cache_promote_pick": (i32, [vp, vp, i32, i32, u64, vp, vp, _P(i32)]),
    "naiwa_cache_slot_table": (i32, [vp, vp]),
    "naiwa_cache_slot_state": (i32, [vp, i32, _P(i32), _P(i32), _P(u64)]),
    "naiwa_cache_hit_counts": (i32, [vp, vp]),
    "naiwa_cache_tick": (i32, [vp, _P(u64)]),
    "naiwa_cache_seed_hits": (i32, [vp, vp]),
    "naiwa_cache_place": (i32, [vp, i32, i32, u64]),
    "naiwa_top_k_ids": (i32, [vp, i32, i32, vp, _P(i32)]),
    "naiwa_union_by_votes": (i32, [vp, vp, i32, vp, i32, _P(i32)]),
    "naiwa_streamed_misses": (i32, [vp, vp, i32, f32, i32, vp, _P(i32)]),
    "naiwa_staging_ring_slots": (i32, []),
    "naiwa_ring_create": (i32, [i32, _P(vp)]),
    "naiwa_ring_destroy": (i32, [vp]),
    "naiwa_ring_acquire": (i32, [vp, i32, _P(i32)]),
    "naiwa_cache_stage": (i32, [vp, vp, vp, i32, i32, f32, vp, vp, vp, _P(i32)]),
    "naiwa_cache_plan": (i32, [vp, i32, vp, vp, i32, i32, f32, _P(StepPlan)]),
    "naiwa_stats_read": (i32, [vp, i32]),
    "naiwa_stats_add": (i32, [vp]),
    # include/naiwa_gguf.h
    "naiwa_prefill_chunk_scratch": (u64, [i32]),
    "naiwa_prefill_activation_bytes": (u64, [i32]),
    "naiwa_prefill_plan": (i32, [u64, u64, i32, i32, u64, u64, i32, _P(i32), _P(i32)]),
    "naiwa_prefill_stream_create": (i32, [_P(PrefillStreamDesc), i64, _P(vp)]),
    "naiwa_prefill_stream_destroy": (i32, [vp]),
    "naiwa_prefill_stream_forward": (i32, [vp, i32, vp, vp, vp, i32, i32, i32, vp, i32, i64]),
    "naiwa_prefill_stream_banks": (i32, [vp, i32, vp, vp, vp]),
    "naiwa_prefill_stream_stats_read": (i32, [vp, _P(PrefillStreamStats)]),
    "naiwa_profile_read": (i32, [C.c_char_p, i32, i32, _P(vp)]),
    "naiwa_profile_destroy": (i32, [vp]),
    "naiwa_profile_layer": (i32, [vp, i32, vp, i32, _P(i32)]),
    "naiwa_profile_info": (i32, [vp, _P(i32), _P(C.c_uint32), _P(C.c_uint32), _P(C.c_uint32)]),
    "naiwa_gguf_open": (i32, [C.c_char_p, _P(vp)]),
    "naiwa_gguf_close": (i32, [vp]),
    "naiwa_gguf_version": (i32, [vp, _P(u32)]),
    "naiwa_gguf_alignment": (i32, [vp, _P(u64)]),
    "naiwa_gguf_tensor_count": (i32, [vp, _P(i32)]),
    "naiwa_gguf_tensor_at": (i32, [vp, i32, vp]),
    "naiwa_gguf_find": (i32, [vp, C.c_char_p, vp]),
    "naiwa_gguf_meta_u64": (i32, [vp, C.c_char_p, _P(u64)]),
    "naiwa_gguf_meta_string": (i32, [vp, C.c_char_p, C.c_char_p, i32, _P(i32)]),
    "naiwa_ggml_type_size": (i32, [i32, _P(i32), _P(i32)]),
    "naiwa_gguf_expert_stack": (i32, [vp, i32, i32, vp]),
}


def lib() -> C.CDLL:
    """The loaded library; raises if it was never built (there is no CPU fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with naiwa-rs_amd/build.py")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != OK:
        raise NaiwaError(rc, what)
