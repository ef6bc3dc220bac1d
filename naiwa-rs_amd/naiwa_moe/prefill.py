"""The whole-layer prefill stream and its memory plan (include/naiwa_prefill.h):
the reference's PrefillStream and plan_with_lend_depth (src/prefill_stream.rs),
with the same names.  The stream runs a chunk's MoE layers over expert stacks in
pinned host memory, one layer upload per buffer of a ring of `depth`, on a copy
stream beside the compute."""
from __future__ import annotations

import ctypes as C

from ._lib import ACT_SILU, PrefillStreamDesc, PrefillStreamStats, check, lib
from .ops import HostExpertStacks, _dev

MIB = 1 << 20
SUB_ROWS = 256
MAX_DEPTH = 4
DEFAULT_DEPTH = 2
CHUNK_HEAD = 256 * MIB
MAX_HEADROOM = 512 * MIB


def chunk_scratch(rows: int) -> int:
    return int(lib().naiwa_prefill_chunk_scratch(rows))


def activation_bytes(chunk: int) -> int:
    return int(lib().naiwa_prefill_activation_bytes(chunk))


def plan_with_lend_depth(free: int, layer_bytes: int, ceiling: int, borrowing: bool, kv_reserve: int,
                         lend_bytes: int, max_depth: int) -> tuple[int, int] | None:
    """(stride, chunk), or None when no chunk fits."""
    stride, chunk = C.c_int(), C.c_int()
    check(lib().naiwa_prefill_plan(free, layer_bytes, ceiling, int(borrowing), kv_reserve, lend_bytes, max_depth,
                                   C.byref(stride), C.byref(chunk)), "prefill_plan")
    return None if chunk.value == 0 else (stride.value, chunk.value)


def plan_with_lend(free, layer_bytes, ceiling, borrowing, kv_reserve, lend_bytes):
    return plan_with_lend_depth(free, layer_bytes, ceiling, borrowing, kv_reserve, lend_bytes, DEFAULT_DEPTH)


def plan_with_reserve(free, layer_bytes, ceiling, borrowing, kv_reserve):
    return plan_with_lend(free, layer_bytes, ceiling, borrowing, kv_reserve, 0)


def plan(free, layer_bytes, ceiling, borrowing):
    return plan_with_reserve(free, layer_bytes, ceiling, borrowing, 0)


class PrefillStream:
    """`depth` device layer buffers fed from per-layer pinned stacks (HostExpertStacks)."""

    def __init__(self, stacks: list[HostExpertStacks], hidden: int, inter: int, dtypes: tuple[int, int, int],
                 depth: int, copy_stream: int):
        n = len(stacks)
        ptrs = [(C.c_void_p * n)(*[s.buffers[p].ptr for s in stacks]) for p in range(3)]
        d = PrefillStreamDesc(n, stacks[0].experts, hidden, inter, *dtypes,
                              C.cast(ptrs[0], C.POINTER(C.c_void_p)), C.cast(ptrs[1], C.POINTER(C.c_void_p)),
                              C.cast(ptrs[2], C.POINTER(C.c_void_p)), depth)
        h = C.c_void_p()
        check(lib().naiwa_prefill_stream_create(C.byref(d), copy_stream, C.byref(h)), "prefill_stream_create")
        self._h, self.depth, self._keep = h, depth, (stacks, ptrs)

    def __del__(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().naiwa_prefill_stream_destroy(self._h)
            self._h = C.c_void_p()

    def forward(self, layer: int, x, expert_ids, weights, T: int, topk: int, out, act: int = ACT_SILU,
                accumulate: bool = False, stream: int = 0) -> None:
        check(lib().naiwa_prefill_stream_forward(self._h, layer, _dev(x), _dev(expert_ids), _dev(weights), T, topk,
                                                 act, _dev(out), 1 if accumulate else 0, stream),
              "prefill_stream_forward")

    def stats(self) -> dict:
        s = PrefillStreamStats()
        check(lib().naiwa_prefill_stream_stats_read(self._h, C.byref(s)), "prefill_stream_stats")
        return {f: int(getattr(s, f)) for f, _ in PrefillStreamStats._fields_}


__all__ = ["PrefillStream", "plan", "plan_with_reserve", "plan_with_lend", "plan_with_lend_depth", "chunk_scratch",
           "activation_bytes", "SUB_ROWS", "MAX_DEPTH", "DEFAULT_DEPTH", "CHUNK_HEAD", "MAX_HEADROOM"]
