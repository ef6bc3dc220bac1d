"""The expert hot path's operators, as the reference's call sites see them.

- ``SlotBank`` / ``LayerBanks``: the slot-indexed GPU expert cache of one layer
  (one ``[slots, N, K]`` bank per projection, src/moe/slot.rs:46-66), filled
  from stacked ``[E, N, K]`` GGUF bytes sliced per expert like
  ``expert_range`` (src/moe/expert.rs:123-145).
- ``indexed_moe_fused_decode``: the call of src/moe/stages/gpu.rs:53-64 with the
  same argument meaning (banks, activations, row-major ``[rows, topk]`` local
  slot ids and weights, activation id); the result is ``[rows, hidden]`` f32.
- ``router_topk`` and ``moe_gather``: routing and grouping on the device.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import (ACT_SILU, BF16, E_UNSUPPORTED, F32, Q4_K, Q8_0, ROUTE_SOFTMAX_TOPK_RENORM, STACK_FUSED,
                   STACK_LAYERED, Bank, Layer, check, lib)
from .device import DeviceBuffer, PinnedBuffer

BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144)}


def row_bytes(dtype: int, k: int) -> int:
    bs, ts = BLOCK[dtype]
    if k % bs:
        raise ValueError(f"K={k} is not divisible by block_size={bs} for dtype {dtype}")
    return (k // bs) * ts


def expert_range(dtype: int, n: int, k: int, e: int) -> range:
    """Byte range of expert e in a stacked [E, N, K] tensor (src/moe/expert.rs:123-145)."""
    stride = n * row_bytes(dtype, k)
    return range(e * stride, (e + 1) * stride)


def slot_stride(dtype: int, n: int, k: int) -> int:
    """Bytes between slots: the projection's bytes rounded up to 256."""
    return (n * row_bytes(dtype, k) + 255) // 256 * 256


class SlotBank:
    """One projection's slot bank on the device."""

    def __init__(self, slots: int, n: int, k: int, dtype: int, buffer: DeviceBuffer | None = None,
                 offset: int = 0, stride: int | None = None):
        self.slots, self.n, self.k, self.dtype = slots, n, k, dtype
        self.stride = slot_stride(dtype, n, k) if stride is None else stride
        self.expert_bytes = n * row_bytes(dtype, k)
        assert self.stride >= self.expert_bytes
        if buffer is None:
            buffer = DeviceBuffer(self.stride * slots)
            offset = 0
        self.buffer, self.offset = buffer, offset
        self.base = buffer.ptr + offset

    def slot_ptr(self, slot: int) -> int:
        if not 0 <= slot < self.slots:
            raise IndexError(f"slot {slot} outside [0, {self.slots})")
        return self.base + slot * self.stride

    def write_slot(self, slot: int, expert_bytes: np.ndarray, stream: int = 0) -> None:
        b = np.ascontiguousarray(expert_bytes, dtype=np.uint8).reshape(-1)
        if b.size != self.expert_bytes:
            raise ValueError(f"expert of {b.size} bytes into a {self.expert_bytes}-byte slot")
        self.buffer.upload(b, stream, offset=self.offset + slot * self.stride)

    def desc(self) -> Bank:
        return Bank(self.base, self.stride, self.slots, self.n, self.k, self.dtype)


class LayerBanks:
    """gate/up/down banks of one layer: gate/up [I, H], down [H, I].  contiguous: one
    allocation whose slot s holds the expert's gate | up | down adjacently (every bank's
    slot stride is the expert's bytes rounded to 256), so an expert moves as one range."""

    def __init__(self, slots: int, hidden: int, inter: int, dtypes: tuple[int, int, int],
                 contiguous: bool = False):
        self.hidden, self.inter, self.slots = hidden, inter, slots
        if not contiguous:
            self.gate = SlotBank(slots, inter, hidden, dtypes[0])
            self.up = SlotBank(slots, inter, hidden, dtypes[1])
            self.down = SlotBank(slots, hidden, inter, dtypes[2])
            return
        pb = [inter * row_bytes(dtypes[0], hidden), inter * row_bytes(dtypes[1], hidden),
              hidden * row_bytes(dtypes[2], inter)]
        stride = (sum(pb) + 255) // 256 * 256
        buf = DeviceBuffer(stride * slots)
        self.gate = SlotBank(slots, inter, hidden, dtypes[0], buf, 0, stride)
        self.up = SlotBank(slots, inter, hidden, dtypes[1], buf, pb[0], stride)
        self.down = SlotBank(slots, hidden, inter, dtypes[2], buf, pb[0] + pb[1], stride)

    def load(self, slot: int, gate: np.ndarray, up: np.ndarray, down: np.ndarray) -> None:
        self.gate.write_slot(slot, gate)
        self.up.write_slot(slot, up)
        self.down.write_slot(slot, down)


def _dev(a) -> int:
    return a.ptr if isinstance(a, DeviceBuffer) else int(a)


class HostExpertStacks:
    """Pinned host copies of one layer's stacked [E, N, K] projections, the sources
    of expert uploads (the reference pins its GGUF stacks, src/host_memory.rs:30-170;
    here they live in pinned allocations, since registering existing memory is not
    available).  Expert e of a projection is at expert_range(e)."""

    def __init__(self, experts: int, hidden: int, inter: int, dtypes: tuple[int, int, int],
                 interleaved: bool = False):
        """interleaved: one pinned allocation holding expert e's gate | up | down adjacently
        at e * stride (stride = the expert's bytes), so an expert uploads as one range."""
        self.experts = experts
        shapes = ((inter, hidden, dtypes[0]), (inter, hidden, dtypes[1]), (hidden, inter, dtypes[2]))
        self.expert_bytes = [n * row_bytes(dt, k) for n, k, dt in shapes]
        if interleaved:
            self.stride = sum(self.expert_bytes)
            self.buffers = [PinnedBuffer(experts * self.stride)]
            offs = [0, self.expert_bytes[0], self.expert_bytes[0] + self.expert_bytes[1]]
            self.ptrs = [self.buffers[0].ptr + o for o in offs]
            self._offs = offs
        else:
            self.stride = 0
            self.buffers = [PinnedBuffer(experts * b) for b in self.expert_bytes]
            self.ptrs = [b.ptr for b in self.buffers]

    def view(self, proj: int) -> np.ndarray:
        """[E, expert_bytes] uint8 view of projection proj (0 gate, 1 up, 2 down); strided
        when the stacks are interleaved."""
        if not self.stride:
            return self.buffers[proj].view().reshape(self.experts, self.expert_bytes[proj])
        whole = self.buffers[0].view().reshape(self.experts, self.stride)
        o = self._offs[proj]
        return whole[:, o:o + self.expert_bytes[proj]]

    def expert_ptrs(self, e: int) -> list[int]:
        if not 0 <= e < self.experts:
            raise IndexError(f"expert {e} outside [0, {self.experts})")
        step = [self.stride or b for b in self.expert_bytes]
        return [p + e * s for p, s in zip(self.ptrs, step)]


def upload_expert(banks: "LayerBanks", slot: int, stacks: HostExpertStacks, expert: int, copy_stream: int,
                  read_fence=None, done=None) -> None:
    """Queue expert `expert`'s three projections into `slot` on copy_stream, after read_fence
    (an Event the compute stream recorded after the slot's last reader) and before done."""
    dst = (C.c_void_p * 3)(banks.gate.slot_ptr(slot), banks.up.slot_ptr(slot), banks.down.slot_ptr(slot))
    src = (C.c_void_p * 3)(*stacks.expert_ptrs(expert))
    sizes = (C.c_size_t * 3)(*stacks.expert_bytes)
    for bank, b in zip((banks.gate, banks.up, banks.down), stacks.expert_bytes):
        if bank.expert_bytes != b:
            raise ValueError("host stacks and slot banks disagree on an expert's size")
    rc = lib().naiwa_upload_expert(dst, src, sizes, copy_stream,
                                   read_fence.handle if read_fence is not None else 0,
                                   done.handle if done is not None else 0)
    check(rc, "naiwa_upload_expert")


COPY_BATCH_MAX = 64


def copy_batch(items, stream: int = 0) -> bool:
    """Queue host -> device copies [(dst, src, bytes), ...] (device pointer, pinned host
    pointer, size; 16-byte aligned) as one kernel on `stream` (naiwa_copy_batch).  False,
    with nothing queued, when a source is not mapped pinned memory or not aligned."""
    if len(items) > COPY_BATCH_MAX:
        raise ValueError(f"at most {COPY_BATCH_MAX} ranges per batch")
    arr = (_lib.Copy * max(1, len(items)))(*[_lib.Copy(d, s, b) for d, s, b in items])
    rc = lib().naiwa_copy_batch(arr, len(items), stream)
    if rc == E_UNSUPPORTED:
        return False
    check(rc, "naiwa_copy_batch")
    return True


def indexed_moe_fused_decode(banks: LayerBanks, x, x_dtype: int, slot_ids, weights, rows: int,
                             topk: int, out, act: int = ACT_SILU, stream: int = 0, accumulate: bool = False) -> None:
    """out[rows, hidden] f32 = sum_j w[t,j] * expert(slot_ids[t,j])(x[t]); all device pointers.
    accumulate: the sums continue from out (naiwa_moe_decode_ex)."""
    g, u, d = banks.gate.desc(), banks.up.desc(), banks.down.desc()
    rc = lib().naiwa_moe_decode_ex(C.byref(g), C.byref(u), C.byref(d), _dev(x), x_dtype,
                                   _dev(slot_ids), _dev(weights), rows, topk, act, _dev(out),
                                   1 if accumulate else 0, stream)
    check(rc, "naiwa_moe_decode_ex")


def moe_prefill(banks: LayerBanks, x, slot_ids, weights, T: int, topk: int, out, act: int = ACT_SILU,
                accumulate: bool = False, stream: int = 0, residual: bool = False) -> None:
    """out[T, hidden] f32 (+)= sum_j w[t,j] * expert(slot_ids[t,j])(x[t]) for a prefill chunk
    (x bf16 [T, hidden]), as grouped MFMA GEMMs; all device pointers.  residual: then also
    x = bf16(x + out) in place."""
    g, u, d = banks.gate.desc(), banks.up.desc(), banks.down.desc()
    flags = (1 if accumulate else 0) | (2 if residual else 0)
    rc = lib().naiwa_moe_prefill(C.byref(g), C.byref(u), C.byref(d), _dev(x), _dev(slot_ids), _dev(weights),
                                 T, topk, act, _dev(out), flags, stream)
    check(rc, "naiwa_moe_prefill")


def router_topk(x, x_dtype: int, W, rows: int, H: int, E: int, k: int, ids_out, w_out,
                mode: int = ROUTE_SOFTMAX_TOPK_RENORM, logits_out=None, stream: int = 0, ld: int = 0) -> None:
    """ld > 0: ids_out / w_out rows ld entries apart (the routed experts in columns 0..k-1)."""
    logits = _dev(logits_out) if logits_out is not None else None
    if ld:
        rc = lib().naiwa_router_topk_ld(_dev(x), x_dtype, _dev(W), None, rows, H, E, k, mode, _dev(ids_out),
                                        _dev(w_out), ld, logits, stream)
        check(rc, "naiwa_router_topk_ld")
        return
    rc = lib().naiwa_router_topk(_dev(x), x_dtype, _dev(W), rows, H, E, k, mode, _dev(ids_out),
                                 _dev(w_out), logits, stream)
    check(rc, "naiwa_router_topk")


def moe_gather(ids, n: int, E: int, perm_out, offsets_out, bad_out=None, stream: int = 0) -> None:
    rc = lib().naiwa_moe_gather(_dev(ids), n, E, _dev(perm_out), _dev(offsets_out),
                                _dev(bad_out) if bad_out is not None else None, stream)
    check(rc, "naiwa_moe_gather")


def layer_desc(router, banks: "LayerBanks", slot_of_expert=None) -> Layer:
    return Layer(_dev(router), banks.gate.desc(), banks.up.desc(), banks.down.desc(),
                 _dev(slot_of_expert) if slot_of_expert is not None else None)


def stack_decode(layers: list, x, rows: int, H: int, E: int, k: int,
                 mode: int = ROUTE_SOFTMAX_TOPK_RENORM, act: int = ACT_SILU, ids_out=None,
                 w_out=None, fused: bool = True, stream: int = 0, y_out=None) -> None:
    """One decode step through every layer: x [rows, H] bf16 (device) updated in place.
    layers: a list of Layer descriptors (layer_desc) or a prebuilt ctypes array.
    y_out: optional f32 device buffer [layers, rows, H] for each layer's MoE output
    before the residual."""
    arr = layers if isinstance(layers, C.Array) else (Layer * len(layers))(*layers)
    rc = lib().naiwa_stack_decode_y(arr, len(arr), _dev(x), rows, H, E, k, mode, act,
                                    _dev(ids_out) if ids_out is not None else None,
                                    _dev(w_out) if w_out is not None else None,
                                    _dev(y_out) if y_out is not None else None,
                                    STACK_FUSED if fused else STACK_LAYERED, stream)
    check(rc, "naiwa_stack_decode")


def stack_status() -> tuple[int, int]:
    a, b = C.c_int(0), C.c_int(0)
    check(lib().naiwa_stack_status(C.byref(a), C.byref(b)), "naiwa_stack_status")
    return a.value, b.value


def synth(dtype: int, seed: int, n: int, out, mean: float = 0.0, std: float = 1.0,
          offset: int = 0, stream: int = 0) -> None:
    """Fill a device buffer with the N(mean, std) stream (seed, offset) as dtype bytes."""
    check(lib().naiwa_synth(dtype, seed, offset, n, mean, std, _dev(out), stream), "naiwa_synth")


__all__ = ["layer_desc", "stack_decode", "stack_status", "synth","SlotBank", "LayerBanks", "indexed_moe_fused_decode", "router_topk", "moe_gather",
           "row_bytes", "expert_range", "slot_stride", "BF16", "F32", "Q4_K", "Q8_0"]
