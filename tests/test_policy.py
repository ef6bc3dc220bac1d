"""Host expert-cache policy (include/naiwa_policy.h) against the reference's own
known answers (src/moe/tests.rs:113-186) and the rules of src/moe/cached_layer.rs,
src/moe/stages/route.rs and src/moe/stages/dma_miss.rs.  Host only: no device."""
import numpy as np
import pytest

from naiwa_moe import policy as P
from naiwa_moe._lib import E_BAD_ID, NaiwaError


def cache_with(resident, hits, slots=None, published=True):
    """A cache whose slot i holds resident[i] (None = empty) and whose hit counts are `hits`."""
    n = len(hits)
    E = max([n] + [e + 1 for e in resident if e is not None])
    c = P.ExpertCache(E, len(resident) if slots is None else slots)
    for s, e in enumerate(resident):
        if e is not None:
            c.place(e, s)
    c.seed_hits(list(hits) + [0] * (E - n))
    return c


# ---- known answers from src/moe/tests.rs --------------------------------------------------

def test_fill_candidate_prefers_hot_unreserved_experts():
    # src/moe/tests.rs:113-131
    assert cache_with([2, None], [0, 5, 9, 5]).fill_candidate() == 1
    assert cache_with([None, None], [0, 0, 0]).fill_candidate() == 0
    assert cache_with([0, 1], [3, 3, 3]).fill_candidate() is None
    assert cache_with([0, 1, None], [1, 1]).fill_candidate() is None


def test_union_by_votes_orders_by_votes_then_rank():
    # src/moe/tests.rs:140-146
    assert P.union_by_votes([[3, 7, 9], [7, 3], [1, 7]]) == [7, 3, 1, 9]
    assert P.union_by_votes([[4, 2]]) == [4, 2]


def test_streamed_misses_ranks_by_total_weight_and_dedups():
    # src/moe/tests.rs:148-162
    misses = [[(1, 0.9), (3, 0.4)], [(3, 0.1), (2, 0.2)]]
    assert P.streamed_misses(misses, 1.0, 3) == [1, 3, 2]
    assert P.streamed_misses(misses, 0.5, 3) == [1, 3]
    assert P.streamed_misses(misses, 1.0, 1) == [1]
    assert P.streamed_misses(misses, 0.0, 3) == []
    assert P.streamed_misses(misses, 1.0, 0) == []


def test_staging_ring_slots_is_fixed():
    # src/moe/tests.rs:164-168
    assert P.staging_ring_slots() == 16


def test_top_k_ids_orders_by_logit_then_index():
    # src/moe/tests.rs:170-174
    assert P.top_k_ids([0.1, 0.9, 0.5, 0.9], 3) == [1, 3, 2]
    assert P.top_k_ids([1.0, 2.0], 5) == [1, 0]


def test_lru_victim_skips_protected_and_prefers_oldest():
    # src/moe/tests.rs:176-186: slots hold experts 10, 11, 12 with last_use 5, 1, 3
    c = P.ExpertCache(13, 3)
    for s, (e, lu) in enumerate([(10, 5), (11, 1), (12, 3)]):
        c.place(e, s, lu)
    assert c.lru_victim([11]) == (12, 2)
    assert c.lru_victim([]) == (11, 1)
    assert c.lru_victim([10, 11, 12]) is None


# ---- the rules the reference states in code ---------------------------------------------------

def test_top_k_ids_uses_the_total_order():
    # f32::total_cmp: -0.0 < +0.0, and ties in value go to the lower index
    assert P.top_k_ids([-0.0, 0.0, -1.0], 3) == [1, 0, 2]
    assert P.top_k_ids([2.0, 2.0, 2.0], 2) == [0, 1]


def test_route_splits_hits_and_misses_and_stamps_ticks():
    c = P.ExpertCache(8, 4)
    c.place(3, 0)
    c.place(5, 2)
    slots = c.route([[3, 1], [5, 3]])
    assert slots.tolist() == [[0, -1], [2, 0]]
    assert c.tick == 1
    assert c.hit_counts().tolist() == [0, 1, 0, 2, 0, 1, 0, 0]
    assert c.slot_state(0) == (3, True, 1) and c.slot_state(2) == (5, True, 1)
    c.route([[1, 6]])
    assert c.tick == 2 and c.slot_state(0)[2] == 1  # not used this step


def test_route_ignores_reserved_slots_and_rejects_bad_ids():
    c = P.ExpertCache(4, 2)
    s = c.admit(2)
    assert s == 0 and c.slot_state(0) == (2, False, 0)
    assert c.route([[2, 1]]).tolist() == [[-1, -1]]  # reserved, not published: a miss
    with pytest.raises(NaiwaError) as err:
        c.route([[1, 4]])
    assert err.value.rc == E_BAD_ID
    assert c.tick == 1  # the failed call changed nothing


def test_admit_takes_the_first_empty_usable_slot_once():
    c = P.ExpertCache(8, 3, usable=2)
    assert c.admit(4) == 0
    assert c.admit(4) is None           # already reserved
    assert c.admit(6) == 1
    assert c.admit(7) is None           # slot 2 is beyond `usable`
    c.publish(0)
    assert c.slot_state(0) == (4, True, 0)
    c.unreserve(1)
    assert c.slot_state(1) == (None, False, 0)
    assert c.admit(7) == 1


def test_replace_evicts_the_lru_outside_protect():
    c = P.ExpertCache(8, 3)
    for s, (e, lu) in enumerate([(1, 4), (2, 2), (3, 9)]):
        c.place(e, s, lu)
    assert c.replace(6, protect=[2]) == 0   # expert 1 (last_use 4) is the oldest unprotected
    assert c.slot_state(0) == (6, False, 4)
    assert c.replace(2) is None             # already resident
    assert c.replace(7) == 1                # slot 0 is unpublished now: expert 2 goes
    assert c.slot_table().tolist() == [-1, -1, -1, 2, -1, -1, -1, -1]


def test_fill_candidate_counts_reserved_slots_as_taken():
    c = cache_with([None, None], [0, 3, 7, 7])
    assert c.fill_candidate() == 2
    c.admit(2)
    assert c.fill_candidate() == 3


def test_promote_pick_rules():
    # 4 usable slots: 0 empty, 1..3 published; tick becomes 2 after one route
    c = P.ExpertCache(16, 4)
    c.place(1, 1, 0)
    c.place(2, 2, 0)
    c.place(3, 3, 0)
    c.route([[1, 9]])       # tick 1: slot 1 used at 1
    c.route([[2, 9]])       # tick 2: slot 2 used at 2 (this step)
    c.seed_hits([0, 0, 0, 0, 5, 4, 3, 0, 9, 6, 0, 0, 0, 0, 0, 0])
    # staged out of order with a duplicate; 6 is cold (3 < 4), 3 is resident
    picks = c.promote_pick([9, 4, 6, 3, 9, 8, 5], cap=3, min_hits=4)
    # id order: 3 resident, 4 -> empty slot 0, 5 -> LRU not used this step: slot 3 (last_use 0),
    # 6 cold, 8 -> slot 1 (last_use 1 < tick 2); cap 3 reached before 9
    assert picks == [(4, 0), (5, 3), (8, 1)]
    for e, s in picks:
        assert c.slot_state(s) == (e, False, c.slot_state(s)[2])
    # nothing left that this step did not read: slot 2 was used at tick 2
    assert c.promote_pick([9], cap=1, min_hits=4) == []
    assert c.promote_pick([10], cap=0) == []


def test_staging_selection_and_ring_positions():
    ring = P.StagingRing()
    assert ring.length == 16
    ids = np.array([[1, 3], [3, 2]], dtype=np.uint32)
    w = np.array([[0.9, 0.4], [0.1, 0.2]], dtype=np.float32)
    slots = np.array([[-1, -1], [-1, 7]], dtype=np.int32)   # (1, 1) pair is a cache hit on slot 7
    staged = ring.stage(ids, w, slots, frac=1.0)
    # misses: 1 (0.9), 3 (0.4 + 0.1): both staged in weight order at positions 0, 1
    assert staged == [(1, 0), (3, 1)]
    F = P.STAGING_RING_FIRST
    assert slots.tolist() == [[F + 0, F + 1], [F + 1, 7]]
    # the cursor advanced by 2; a 15-expert step wraps
    ids2 = np.arange(15, dtype=np.uint32).reshape(15, 1)
    slots2 = np.full((15, 1), -1, dtype=np.int32)
    staged2 = ring.stage(ids2, np.linspace(1.0, 0.1, 15, dtype=np.float32).reshape(15, 1), slots2, 1.0)
    assert [p for _, p in staged2] == [(2 + i) % 16 for i in range(15)]
    # frac 0: nothing staged, slots untouched
    slots3 = np.full((1, 2), -1, dtype=np.int32)
    assert ring.stage(ids[:1], w[:1], slots3, 0.0) == [] and slots3.tolist() == [[-1, -1]]


def test_streamed_misses_sums_in_row_major_f32_order():
    # 0.1 + 0.2 + 0.3 in f32 in that order, against 0.6 exactly: the f32 sum decides the ranking
    w = [np.float32(0.1), np.float32(0.2), np.float32(0.3)]
    s = np.float32(np.float32(w[0] + w[1]) + w[2])
    misses = [[(5, float(w[0]))], [(5, float(w[1]))], [(5, float(w[2]))], [(4, float(s))]]
    # equal f32 sums: ties go to the lower id
    assert P.streamed_misses(misses, 1.0, 2) == [4, 5]


def test_stats_accumulate_and_reset():
    P.stats(reset=True)
    P.stats_add(hits=3, staged=2, pcie_bytes=100)
    P.stats_add(hits=1)
    s = P.stats(reset=True)
    assert s["hits"] == 4 and s["staged"] == 2 and s["pcie_bytes"] == 100 and s["misses"] == 0
    assert P.stats()["hits"] == 0


# ---- the step plan: route + stage without their side effects ------------------------------

def _state(c, ring):
    slots = [c.slot_state(s) for s in range(c.slots)]
    return c.tick, c.hit_counts().tolist(), slots, ring.acquire(0)


@pytest.mark.parametrize("frac", [0.0, 0.5, 1.0])
def test_plan_predicts_route_and_stage_and_changes_nothing(frac):
    """naiwa_cache_plan reports the hits, staged pairs, staged experts and CPU pairs that
    naiwa_cache_route followed by naiwa_cache_stage then produce, over a run of random
    Zipf-like steps, and leaves the tick, the hit counts, every slot's state and the ring
    cursor exactly as they were (the partial-cache step refuses a step it cannot finish
    with it, before anything moves)."""
    rng = np.random.default_rng(7)
    E, slots, k, rows = 64, 12, 6, 3
    c = P.ExpertCache(E, slots)
    for s in range(slots):
        c.place(int(s * 5 % E), s)
    ring = P.StagingRing(8)
    pop = 1.0 / np.arange(1, E + 1) ** 1.1
    pop /= pop.sum()
    for step in range(30):
        ids = np.stack([rng.choice(E, size=k, replace=False, p=pop) for _ in range(rows)]).astype(np.uint32)
        w = rng.random((rows, k)).astype(np.float32)
        w[0, 0] = 0.0  # a zero weight still counts as a pair of its kind
        before = _state(c, ring)
        plan = c.plan(ids, w, ring.length, frac)
        assert _state(c, ring) == before, step
        got = c.route(ids)
        slots_io = np.array(got, dtype=np.int32).reshape(rows, k)
        staged = ring.stage(ids, w, slots_io, frac)
        hits = int((np.array(got) >= 0).sum())
        in_ring = int((slots_io >= P.STAGING_RING_FIRST).sum())
        cpu = int((slots_io < 0).sum())
        assert plan == {"hits": hits, "staged": in_ring, "staged_experts": len(staged), "cpu": cpu}, (step, plan)
        assert hits + in_ring + cpu == rows * k


def test_plan_rejects_bad_ids_without_changing_state():
    c = P.ExpertCache(8, 2)
    ring = P.StagingRing(4)
    before = _state(c, ring)
    with pytest.raises(NaiwaError) as e:
        c.plan(np.array([[1, 9]], dtype=np.uint32), np.ones((1, 2), np.float32), ring.length, 1.0)
    assert e.value.rc == E_BAD_ID
    assert _state(c, ring) == before


def test_cached_layer_rejects_overlapping_host_stacks():
    """naiwa_cached_layer_create refuses a negative host_expert_stride, or a positive
    one shorter than a projection (the experts would overlap in the host stacks), with
    NAIWA_E_INVALID before it touches a device: every pointer here is made up."""
    import ctypes as C
    from naiwa_moe import Q4_K
    from naiwa_moe._lib import Bank, CachedLayerDesc, E_INVALID, lib
    L = lib()
    E, H, I, usable = 8, 256, 256, 2
    ring = P.StagingRing()
    proj = L.naiwa_projection_bytes(Q4_K, I, H)                  # 36,864 B a projection here
    stride = (proj + 255) // 256 * 256
    fake = 0x7f0000000000
    bank = lambda n, k: Bank(fake, stride, usable + ring.length, n, k, Q4_K)
    for host_stride in (-1, proj - 16, 1):
        d = CachedLayerDesc(fake, None, bank(I, H), bank(I, H), bank(H, I), fake, fake, fake, E, 2, H, I, usable,
                            0, 0, host_stride)
        h = C.c_void_p()
        rc = L.naiwa_cached_layer_create(C.byref(d), ring._h, ring.length, 0, C.byref(h))
        assert rc == E_INVALID, (host_stride, rc)
        assert not h.value
