"""Host-side expert-cache policy over include/naiwa_policy.h.

Mirrors the reference's CachedLayer residency rules (src/moe/cached_layer.rs,
src/moe/stages/route.rs, src/moe/stages/dma_miss.rs, src/moe/staging.rs) with
the same names: route / fill_candidate / lru_victim / admit / replace /
promote_staged selection, top_k_ids, union_by_votes, streamed_misses and the
staging ring.  Everything runs in the C++ library on the host.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import (STAGING_RING_FIRST, STATS_FIELDS, CacheStats, CachedLayerDesc, CachedStep, LookaheadStep, check,
                   lib)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ptr(a: np.ndarray):
    return a.ctypes.data if a.size else None


class ExpertCache:
    """One layer's slot cache: `slots` slots, the first `usable` of which hold experts."""

    def __init__(self, num_experts: int, slots: int, usable: int | None = None, _borrowed=None):
        self.num_experts = num_experts
        self.slots = slots
        self._owned = _borrowed is None
        if _borrowed is not None:
            self._h = _borrowed
            return
        h = C.c_void_p()
        check(lib().naiwa_cache_create(num_experts, slots, slots if usable is None else usable, C.byref(h)),
              "cache_create")
        self._h = h

    def __del__(self):
        if getattr(self, "_owned", False) and getattr(self, "_h", None) and self._h.value:
            lib().naiwa_cache_destroy(self._h)
            self._h = C.c_void_p()

    def route(self, ids) -> np.ndarray:
        """Route::submit: returns slot per (row, k) pair, -1 for a miss."""
        ids = _u32(ids)
        rows, k = ids.shape
        out = np.empty((rows, k), dtype=np.int32)
        check(lib().naiwa_cache_route(self._h, _ptr(ids), rows, k, _ptr(out)), "cache_route")
        return out

    def fill_candidate(self) -> int | None:
        e, found = C.c_int(), C.c_int()
        check(lib().naiwa_cache_fill_candidate(self._h, C.byref(e), C.byref(found)), "fill_candidate")
        return e.value if found.value else None

    def lru_victim(self, protect=()) -> tuple[int, int] | None:
        p = _i32(list(protect))
        e, s, found = C.c_int(), C.c_int(), C.c_int()
        check(lib().naiwa_cache_lru_victim(self._h, _ptr(p), p.size, C.byref(e), C.byref(s), C.byref(found)),
              "lru_victim")
        return (e.value, s.value) if found.value else None

    def admit(self, expert: int) -> int | None:
        s = C.c_int()
        check(lib().naiwa_cache_admit(self._h, expert, C.byref(s)), "admit")
        return s.value if s.value >= 0 else None

    def replace(self, expert: int, protect=()) -> int | None:
        p = _i32(list(protect))
        s = C.c_int()
        check(lib().naiwa_cache_replace(self._h, expert, _ptr(p), p.size, C.byref(s)), "replace")
        return s.value if s.value >= 0 else None

    def publish(self, slot: int) -> None:
        check(lib().naiwa_cache_publish(self._h, slot), "publish")

    def unreserve(self, slot: int) -> None:
        check(lib().naiwa_cache_unreserve(self._h, slot), "unreserve")

    def promote_pick(self, staged, cap: int = 1, min_hits: int = 4) -> list[tuple[int, int]]:
        st = _u32(list(staged))
        ex = np.empty(max(cap, 1), dtype=np.int32)
        sl = np.empty(max(cap, 1), dtype=np.int32)
        n = C.c_int()
        check(lib().naiwa_cache_promote_pick(self._h, _ptr(st), st.size, cap, min_hits, _ptr(ex), _ptr(sl),
                                             C.byref(n)), "promote_pick")
        return [(int(ex[i]), int(sl[i])) for i in range(n.value)]

    def slot_table(self) -> np.ndarray:
        out = np.empty(self.num_experts, dtype=np.int32)
        check(lib().naiwa_cache_slot_table(self._h, _ptr(out)), "slot_table")
        return out

    def slot_state(self, slot: int) -> tuple[int | None, bool, int]:
        e, pub, lu = C.c_int(), C.c_int(), C.c_uint64()
        check(lib().naiwa_cache_slot_state(self._h, slot, C.byref(e), C.byref(pub), C.byref(lu)), "slot_state")
        return (e.value if e.value >= 0 else None, bool(pub.value), lu.value)

    def hit_counts(self) -> np.ndarray:
        out = np.empty(self.num_experts, dtype=np.uint64)
        check(lib().naiwa_cache_hit_counts(self._h, _ptr(out)), "hit_counts")
        return out

    def seed_hits(self, counts) -> None:
        c = np.ascontiguousarray(np.asarray(counts, dtype=np.uint64))
        assert c.size == self.num_experts
        check(lib().naiwa_cache_seed_hits(self._h, _ptr(c)), "seed_hits")

    @property
    def tick(self) -> int:
        t = C.c_uint64()
        check(lib().naiwa_cache_tick(self._h, C.byref(t)), "tick")
        return t.value

    def place(self, expert: int, slot: int, last_use: int = 0) -> None:
        check(lib().naiwa_cache_place(self._h, expert, slot, last_use), "place")

    def plan(self, ids, w, ring_len: int, frac: float) -> dict:
        """naiwa_cache_plan: the split route + stage would make, with no state changed."""
        from ._lib import StepPlan
        ids, w = _u32(ids), _f32(w)
        rows, k = ids.shape
        out = StepPlan()
        check(lib().naiwa_cache_plan(self._h, ring_len, _ptr(ids), _ptr(w), rows, k, frac, C.byref(out)),
              "cache_plan")
        return {f: getattr(out, f) for f, _ in StepPlan._fields_}


class StagingRing:
    """The round-robin staging ring (ring slots are NAIWA_STAGING_RING_FIRST + position)."""

    def __init__(self, length: int | None = None):
        self.length = staging_ring_slots() if length is None else length
        h = C.c_void_p()
        check(lib().naiwa_ring_create(self.length, C.byref(h)), "ring_create")
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().naiwa_ring_destroy(self._h)
            self._h = C.c_void_p()

    def acquire(self, n: int) -> int:
        start = C.c_int()
        check(lib().naiwa_ring_acquire(self._h, n, C.byref(start)), "ring_acquire")
        return start.value

    def stage(self, ids, w, slots, frac: float) -> list[tuple[int, int]]:
        """stage_misses selection: updates `slots` in place (staged misses become ring slots) and
        returns (expert, ring position) per staged expert."""
        ids, w = _u32(ids), _f32(w)
        rows, k = ids.shape
        assert slots.dtype == np.int32 and slots.flags.c_contiguous and slots.shape == (rows, k)
        chosen = np.empty(self.length, dtype=np.uint32)
        pos = np.empty(self.length, dtype=np.int32)
        n = C.c_int()
        check(lib().naiwa_cache_stage(self._h, _ptr(ids), _ptr(w), rows, k, frac, _ptr(slots), _ptr(chosen),
                                      _ptr(pos), C.byref(n)), "cache_stage")
        return [(int(chosen[i]), int(pos[i])) for i in range(n.value)]


def _host_ptrs(stacks) -> list[int]:
    """The host pointers of expert 0's gate, up and down projections."""
    ptrs = getattr(stacks, "ptrs", None)
    return list(ptrs) if ptrs is not None else [b.ptr for b in stacks.buffers]


class CachedLayer:
    """One layer's decode step over a partial cache (include/naiwa_cached.h): the reference's
    CachedExperts::forward for decode rows, with PCIe staging and promotion."""

    def __init__(self, router, banks, stacks, num_experts: int, top_k: int, usable: int, ring: "StagingRing",
                 copy_stream: int, mode: int = 0, act: int = 0, router_bias=None):
        from .ops import _dev
        d = CachedLayerDesc(_dev(router), _dev(router_bias) if router_bias is not None else None,
                            banks.gate.desc(), banks.up.desc(), banks.down.desc(),
                            *_host_ptrs(stacks), num_experts, top_k, banks.hidden, banks.inter, usable,
                            mode, act, getattr(stacks, "stride", 0))
        h = C.c_void_p()
        check(lib().naiwa_cached_layer_create(C.byref(d), ring._h, ring.length, copy_stream, C.byref(h)),
              "cached_layer_create")
        self._h, self.top_k, self.usable = h, top_k, usable
        self._keep = (router, banks, stacks, ring, router_bias)
        c = C.c_void_p()
        check(lib().naiwa_cached_layer_cache(h, C.byref(c)), "cached_layer_cache")
        self.cache = ExpertCache(num_experts, usable, _borrowed=c)

    def __del__(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().naiwa_cached_layer_destroy(self._h)
            self._h = C.c_void_p()

    def fill(self, expert: int) -> int | None:
        s = C.c_int()
        check(lib().naiwa_cached_layer_fill(self._h, expert, C.byref(s)), "cached_layer_fill")
        return s.value if s.value >= 0 else None

    def seed(self, experts, fill_share: float = 1.0) -> int:
        """Profile seeding: the first round(usable * fill_share) ranked experts, admitted in order."""
        e = _u32(list(experts))
        n = C.c_int()
        check(lib().naiwa_cached_layer_seed(self._h, _ptr(e), e.size, fill_share, C.byref(n)), "cached_layer_seed")
        return n.value

    def forward(self, x, rows: int, out, pcie_frac: float = 1.0, promote_cap: int = 1, min_hits: int = 4,
                stream: int = 0) -> dict:
        from .ops import _dev
        info = CachedStep()
        check(lib().naiwa_cached_layer_forward(self._h, _dev(x), rows, _dev(out), pcie_frac, promote_cap, min_hits,
                                               stream, C.byref(info)), "cached_layer_forward")
        return {f: getattr(info, f) for f, _ in CachedStep._fields_}

    def forward_ahead(self, next_layer: "CachedLayer", x, rows: int, out, lookahead_swaps: int = 2,
                      pcie_frac: float = 1.0, promote_cap: int = 1, min_hits: int = 4,
                      stream: int = 0) -> tuple[dict, dict]:
        """forward, plus next_layer's lookahead on the same x (one routing read-back)."""
        from .ops import _dev
        info, ahead = CachedStep(), LookaheadStep()
        check(lib().naiwa_cached_layer_forward_ahead(self._h, next_layer._h, lookahead_swaps, _dev(x), rows, _dev(out),
                                                     pcie_frac, promote_cap, min_hits, stream, C.byref(info),
                                                     C.byref(ahead)), "cached_layer_forward_ahead")
        return ({f: getattr(info, f) for f, _ in CachedStep._fields_},
                {f: getattr(ahead, f) for f, _ in LookaheadStep._fields_})

    def prefetch_predicted(self, x, rows: int, lookahead_swaps: int = 2, stream: int = 0) -> dict:
        """This layer's lookahead on the previous layer's activation x."""
        from .ops import _dev
        ahead = LookaheadStep()
        check(lib().naiwa_cached_layer_prefetch(self._h, _dev(x), rows, lookahead_swaps, stream, C.byref(ahead)),
              "cached_layer_prefetch")
        return {f: getattr(ahead, f) for f, _ in LookaheadStep._fields_}

    @staticmethod
    def stack_forward(layers: list["CachedLayer"], x, rows: int, y, pcie_frac: float = 1.0, promote_cap: int = 1,
                      min_hits: int = 4, lookahead_swaps: int = -1, stream: int = 0) -> tuple[dict, dict]:
        """One decode step through the layers in order (naiwa_cached_stack_forward): each layer's
        partial-cache step on x into y, then x = bf16(x + y); lookahead_swaps >= 0 adds the
        lookahead.  Returns the summed step and lookahead reports."""
        from .ops import _dev
        arr = (C.c_void_p * len(layers))(*[layer._h.value for layer in layers])
        info, ahead = CachedStep(), LookaheadStep()
        check(lib().naiwa_cached_stack_forward(arr, len(layers), _dev(x), rows, _dev(y), pcie_frac, promote_cap,
                                               min_hits, lookahead_swaps, stream, C.byref(info), C.byref(ahead)),
              "cached_stack_forward")
        return ({f: getattr(info, f) for f, _ in CachedStep._fields_},
                {f: getattr(ahead, f) for f, _ in LookaheadStep._fields_})

    def predicted(self) -> list[int]:
        out = np.empty(max(self.cache.num_experts, 1), dtype=np.uint32)
        n = C.c_int()
        check(lib().naiwa_cached_layer_predicted(self._h, _ptr(out), out.size, C.byref(n)), "cached_layer_predicted")
        return [int(v) for v in out[:n.value]]

    def set_upload_sync(self, mode: int) -> None:
        """UPLOAD_SYNC_EVENT (0) or UPLOAD_SYNC_POLL (1, the default): how staged uploads
        complete into the expert pass."""
        check(lib().naiwa_cached_layer_set_upload_sync(self._h, mode), "cached_layer_set_upload_sync")

    def set_upload_path(self, path: int) -> None:
        """UPLOAD_PATH_KERNEL (0, the default) or UPLOAD_PATH_DMA (1): how staged uploads travel."""
        check(lib().naiwa_cached_layer_set_upload_path(self._h, path), "cached_layer_set_upload_path")

    def set_cpu_misses(self, on: bool) -> None:
        """Misses the ring does not take run on the CPU (default), or such a step is refused."""
        check(lib().naiwa_cached_layer_set_cpu_misses(self._h, 1 if on else 0), "cached_layer_set_cpu_misses")

    def upload_timeouts(self) -> int:
        n = C.c_uint32()
        check(lib().naiwa_cached_layer_upload_timeouts(self._h, C.byref(n)), "cached_layer_upload_timeouts")
        return n.value

    def routing(self, rows: int) -> tuple[np.ndarray, np.ndarray]:
        ids = np.empty((rows, self.top_k), dtype=np.uint32)
        w = np.empty((rows, self.top_k), dtype=np.float32)
        check(lib().naiwa_cached_layer_routing(self._h, _ptr(ids), _ptr(w), ids.size), "cached_layer_routing")
        return ids, w


class ExpertProfile:
    """The expert-cache profile (src/moe/profile.rs): per layer, its experts best first."""

    # the reference reads with generous bounds and filters to the model (src/load.rs:25-29)
    LAYERS, EXPERTS = 128, 1024

    def __init__(self, path, num_layers: int = LAYERS, num_experts: int = EXPERTS):
        h = C.c_void_p()
        check(lib().naiwa_profile_read(str(path).encode(), num_layers, num_experts, C.byref(h)), "profile_read")
        self._h, self.num_experts = h, num_experts
        pairs = C.c_int()
        fl, fe, fp = C.c_uint32(), C.c_uint32(), C.c_uint32()
        check(lib().naiwa_profile_info(h, C.byref(pairs), C.byref(fl), C.byref(fe), C.byref(fp)), "profile_info")
        self.pairs = pairs.value
        self.source = f"{path} ({fl.value}x{fe.value}, {fp.value} ranked pairs)"

    def __del__(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().naiwa_profile_destroy(self._h)
            self._h = C.c_void_p()

    def layer(self, layer: int) -> list[int]:
        out = np.empty(max(self.num_experts, 1), dtype=np.uint32)
        n = C.c_int()
        check(lib().naiwa_profile_layer(self._h, layer, _ptr(out), out.size, C.byref(n)), "profile_layer")
        return [int(v) for v in out[:n.value]]


def write_profile(path, pairs, layers: int, experts: int, slots: int | None = None) -> None:
    """Write a profile file: the ranking (layer, expert) best first, then the rank table."""
    import struct
    n = len(pairs)
    out = bytearray(b"STRP" + struct.pack("<5I", 1, layers, experts, n if slots is None else slots, n))
    for l, e in pairs:
        out += struct.pack("<HH", l, e)
    table = np.full((layers, experts), -1, dtype="<i4")
    for r, (l, e) in enumerate(pairs):
        if l < layers and e < experts and table[l, e] < 0:
            table[l, e] = r
    out += table.tobytes()
    with open(path, "wb") as f:
        f.write(bytes(out))


def hit_rate(s: dict) -> float:
    """CacheStats::hit_rate (src/stats/cache.rs:121-124): hits / (hits + misses)."""
    return s["hits"] / max(s["hits"] + s["misses"], 1)


def staging_ring_slots() -> int:
    return int(lib().naiwa_staging_ring_slots())


def top_k_ids(logits, k: int) -> list[int]:
    x = _f32(logits)
    out = np.empty(max(min(k, x.size), 1), dtype=np.uint32)
    n = C.c_int()
    check(lib().naiwa_top_k_ids(_ptr(x), x.size, k, _ptr(out), C.byref(n)), "top_k_ids")
    return [int(v) for v in out[:n.value]]


def union_by_votes(rankings) -> list[int]:
    rankings = [list(r) for r in rankings]
    flat = _u32([e for r in rankings for e in r])
    lens = _i32([len(r) for r in rankings])
    out = np.empty(max(flat.size, 1), dtype=np.uint32)
    n = C.c_int()
    check(lib().naiwa_union_by_votes(_ptr(flat), _ptr(lens), len(rankings), _ptr(out), out.size, C.byref(n)),
          "union_by_votes")
    return [int(v) for v in out[:n.value]]


def streamed_misses(misses, frac: float, cap: int) -> list[int]:
    """misses: rows of (id, weight) pairs, as the reference's Vec<Vec<(u32, f32)>>."""
    flat = [p for row in misses for p in row]
    ids = _u32([p[0] for p in flat])
    w = _f32([p[1] for p in flat])
    out = np.empty(max(cap, 1), dtype=np.uint32)
    n = C.c_int()
    check(lib().naiwa_streamed_misses(_ptr(ids), _ptr(w), ids.size, frac, cap, _ptr(out), C.byref(n)),
          "streamed_misses")
    return [int(v) for v in out[:n.value]]


def stats(reset: bool = False) -> dict[str, int]:
    s = CacheStats()
    check(lib().naiwa_stats_read(C.byref(s), int(reset)), "stats_read")
    return {f: int(getattr(s, f)) for f in STATS_FIELDS}


def stats_add(**delta: int) -> None:
    s = CacheStats(**{f: int(delta.get(f, 0)) for f in STATS_FIELDS})
    check(lib().naiwa_stats_add(C.byref(s)), "stats_add")


__all__ = ["ExpertCache", "StagingRing", "CachedLayer", "ExpertProfile", "STAGING_RING_FIRST", "staging_ring_slots",
           "top_k_ids", "union_by_votes", "streamed_misses", "stats", "stats_add", "hit_rate", "write_profile"]


UPLOAD_SYNC_EVENT = 0
UPLOAD_SYNC_POLL = 1
UPLOAD_PATH_KERNEL = 0
UPLOAD_PATH_DMA = 1


def cpu_moe_decode(gate, up, down, dtypes, hidden: int, inter: int, xs, ids, w, act: int = 0) -> np.ndarray:
    """naiwa_cpu_moe_decode: the CPU expert path (fused_moe_decode contract) over host
    stacks gate/up [E, inter, row bytes] and down [E, hidden, row bytes]; xs f32 [rows,
    hidden]; ids/w [rows, width].  Returns f32 [rows, hidden]."""
    from ._lib import HostExperts
    g, u, d = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down))
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ids, w = _u32(ids), _f32(w)
    rows, width = ids.shape
    ex = HostExperts(g.ctypes.data, u.ctypes.data, d.ctypes.data, 0, 0, 0, dtypes[0], dtypes[1], dtypes[2],
                     g.shape[0], hidden, inter)
    out = np.empty((rows, hidden), dtype=np.float32)
    check(lib().naiwa_cpu_moe_decode(C.byref(ex), _ptr(xs), _ptr(ids), _ptr(w), rows, width, act, _ptr(out)),
          "cpu_moe_decode")
    return out

