"""naiwa_moe: host binding of the gfx950 MoE expert hot path (libnaiwa_moe.so).

Mirrors the reference's moe / doorbell / executor interfaces over the C ABI of
include/naiwa_moe.h.  Nothing here computes on the CPU: every operator calls
the HIP library, which must be built (naiwa-rs_amd/build.py).
"""
from ._lib import (ACT_GELU_PYTORCH_TANH, ACT_SILU, BF16, E_BAD_ID, E_DEVICE, E_FORMAT, E_INVALID, E_IO,
                   E_NOMEM, E_NOT_FOUND, E_TIMEOUT, E_TOO_LARGE, E_UNSUPPORTED, F16, F32, Q4_K, Q8_0,
                   ROUTE_SOFTMAX_TOPK, ROUTE_SOFTMAX_TOPK_RENORM, ROUTE_TOPK_SOFTMAX, LIB_PATH,
                   NaiwaError, lib)
from .device import DeviceBuffer, Event, PinnedBuffer, Stream, device_count, device_info, mem_info, synchronize
from . import doorbells, gguf, policy, prefill
from .ops import (HostExpertStacks, LayerBanks, SlotBank, copy_batch, expert_range, indexed_moe_fused_decode,
                  layer_desc, moe_gather, moe_prefill, router_topk, row_bytes, slot_stride, stack_decode, stack_status,
                  synth, upload_expert)

__all__ = [
    "ACT_GELU_PYTORCH_TANH", "ACT_SILU", "BF16", "F16", "F32", "Q4_K", "Q8_0", "E_BAD_ID", "E_DEVICE",
    "E_FORMAT", "E_INVALID", "E_IO", "E_NOMEM", "E_NOT_FOUND", "E_TIMEOUT", "E_TOO_LARGE", "E_UNSUPPORTED",
    "ROUTE_SOFTMAX_TOPK", "ROUTE_SOFTMAX_TOPK_RENORM", "ROUTE_TOPK_SOFTMAX", "LIB_PATH",
    "NaiwaError", "lib", "DeviceBuffer", "Event", "PinnedBuffer", "Stream", "device_count",
    "device_info", "mem_info", "synchronize", "LayerBanks", "SlotBank", "expert_range",
    "indexed_moe_fused_decode", "moe_gather", "moe_prefill", "router_topk", "row_bytes", "slot_stride",
    "layer_desc", "stack_decode", "stack_status", "synth", "policy", "doorbells", "gguf", "prefill", "HostExpertStacks", "upload_expert",
    "copy_batch",
]
