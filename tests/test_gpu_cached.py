"""GPU parity of the partial-cache decode step (include/naiwa_cached.h): device
routing with a per-expert bias is bit-exact with the oracle, the hit/miss split
and staging follow the host policy, staged experts are uploaded byte-exactly into
their ring slots, promotion moves them into the cache, the lookahead loads the
next layer's predicted experts by the reference's admit/replace rules, and every
step's expert output is within the 1e-2 relative bar of the oracle over the same
routed set."""
import numpy as np
import pytest

import oracle as O
import synthetic as S

pytestmark = pytest.mark.gpu
TOL = 1e-2


def zipf_bias(E: int, s: float, seed: int) -> np.ndarray:
    ranks = np.random.default_rng(seed).permutation(E) + 1
    p = ranks.astype(np.float64) ** -s
    return np.log(p / p.sum()).astype(np.float32)


def make_layer(nm, seed, E, H, I, k, usable, ring, copy, dt=(O.Q4_K,) * 3, bias_scale=1.0):
    g, u, d, r = S.layer(seed, E, H, I, dt)
    stacks = nm.HostExpertStacks(E, H, I, dt)
    for p, src in enumerate((g, u, d)):
        stacks.view(p)[:] = src.reshape(E, -1)
    banks = nm.LayerBanks(usable + ring.length, H, I, dt)
    router = nm.DeviceBuffer.from_array(r)
    bias = zipf_bias(E, 1.1, seed) * np.float32(bias_scale)
    bias_d = nm.DeviceBuffer.from_array(bias)
    layer = nm.policy.CachedLayer(router, banks, stacks, E, k, usable, ring, copy.handle,
                                  mode=O.ROUTE_SOFTMAX_TOPK_RENORM, router_bias=bias_d)
    host = (g, u, d, r, bias, dt, I)
    return layer, banks, stacks, host


def oracle_step(host, x_bf16, E, k, H):
    g, u, d, r, bias, dt, I = host
    xf = O.from_bf16(x_bf16)
    logits = (O.router_logits(xf, r).astype(np.float32) + bias).astype(np.float32)
    ids, w = O.topk(logits, k, O.ROUTE_SOFTMAX_TOPK_RENORM)
    gs, us, ds = O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I)
    return ids, w, O.fused_moe_decode(gs, us, ds, xf, ids, w)


def test_cached_layer_steps_match_the_oracle(gpu):
    nm = gpu
    E, H, I, k, usable, rows = 16, 256, 256, 4, 4, 2
    copy = nm.Stream()
    stream = nm.Stream()
    ring = nm.policy.StagingRing()
    layer, banks, stacks, host = make_layer(nm, 1200, E, H, I, k, usable, ring, copy)
    for e in range(usable):
        assert layer.fill(e) == e
    assert layer.cache.slot_table()[:usable].tolist() == list(range(usable))
    out = nm.DeviceBuffer(rows * H * 4)
    nm.policy.stats(reset=True)
    total = {"hits": 0, "staged": 0, "staged_experts": 0, "promoted": 0, "pcie_bytes": 0}
    per_expert = sum(stacks.expert_bytes)
    for step in range(6):
        print(f"[cached step {step}]", flush=True)
        x = S.activations_bf16(1300 + step, rows, H)
        xd = nm.DeviceBuffer.from_array(x)
        resident_before = layer.cache.slot_table()
        info = layer.forward(xd, rows, out, pcie_frac=1.0, promote_cap=1, min_hits=1, stream=stream.handle)
        stream.sync()
        ids, w = layer.routing(rows)
        want_ids, want_w, want = oracle_step(host, x, E, k, H)
        assert np.array_equal(ids, want_ids), (step, ids, want_ids)
        assert np.allclose(w, want_w, rtol=1e-5, atol=1e-7)
        hits = int(sum(resident_before[i] >= 0 for i in ids.reshape(-1)))
        assert info["hits"] == hits and info["hits"] + info["staged"] == rows * k
        assert info["staged_experts"] == len(set(int(i) for i in ids.reshape(-1) if resident_before[i] < 0))
        assert info["pcie_bytes"] == info["staged_experts"] * per_expert
        got = out.download(np.float32).reshape(rows, H)
        err = S.max_rel_err(got, want)
        print(f"  hits={info['hits']} staged={info['staged']} promoted={info['promoted']} err={err:.3e}",
              flush=True)
        assert err < TOL
        for key in total:
            total[key] += info[key]
    st = nm.policy.stats()
    assert st["hits"] == total["hits"] and st["staged"] == total["staged"]
    assert st["pcie_bytes"] == total["pcie_bytes"] and st["promotions"] == total["promoted"]
    assert total["promoted"] > 0   # min_hits 1: every step promotes one staged expert
    # promoted experts are resident and all three projections hold the expert's bytes
    check_resident_bytes(layer, banks, stacks)


def check_resident_bytes(layer, banks, stacks):
    table = layer.cache.slot_table()
    for e in np.nonzero(table >= 0)[0]:
        s = int(table[e])
        for proj, bank in enumerate((banks.gate, banks.up, banks.down)):
            got = bank.buffer.download(np.uint8, count=bank.expert_bytes, offset=bank.offset + s * bank.stride)
            assert np.array_equal(got, stacks.view(proj)[e]), (e, s, proj)


def test_staged_bytes_land_in_their_ring_slot(gpu):
    nm = gpu
    E, H, I, k, usable, rows = 8, 256, 256, 2, 2, 1
    copy, stream = nm.Stream(), nm.Stream()
    ring = nm.policy.StagingRing()
    layer, banks, stacks, host = make_layer(nm, 1400, E, H, I, k, usable, ring, copy, dt=(O.Q8_0,) * 3)
    out = nm.DeviceBuffer(rows * H * 4)
    x = S.activations_bf16(1401, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    info = layer.forward(xd, rows, out, pcie_frac=1.0, promote_cap=0, stream=stream.handle)
    stream.sync()
    ids, _ = layer.routing(rows)
    assert info["hits"] == 0 and info["staged_experts"] == len(set(ids.reshape(-1).tolist()))
    # a fresh ring starts at position 0: the staged experts sit in bank slots usable + i
    want_ids, want_w, want = oracle_step(host, x, E, k, H)
    assert np.array_equal(ids, want_ids)
    assert S.max_rel_err(out.download(np.float32).reshape(rows, H), want) < TOL
    # streamed_misses order: by summed weight (rows = 1: weight order)
    order = nm.policy.streamed_misses([[(int(i), float(v)) for i, v in zip(ids[0], want_w[0])]], 1.0, 16)
    for pos, e in enumerate(order):
        for proj, bank in enumerate((banks.gate, banks.up, banks.down)):
            got = bank.buffer.download(np.uint8, count=bank.expert_bytes, offset=bank.offset + (usable + pos) * bank.stride)
            assert np.array_equal(got, stacks.view(proj)[e])


class SlotModel:
    """The reference's residency rules for a cache with no promotions
    (src/moe/stages/route.rs:19-158, src/moe/cached_layer.rs:401-410, 1056-1101):
    route bumps the tick and touches hits; admit takes the first empty slot;
    replace takes the resident with the smallest (last_use, expert) outside the
    protected set; a loaded slot is published with last_use = tick."""

    def __init__(self, usable: int):
        self.expert = [None] * usable
        self.last = [0] * usable
        self.tick = 0

    def resident(self, e):
        return e in self.expert

    def route(self, ids):
        self.tick += 1
        hits = 0
        for e in ids:
            if e in self.expert:
                self.last[self.expert.index(e)] = self.tick
                hits += 1
        return hits

    def admit(self, e):
        if e in self.expert or None not in self.expert:
            return False
        s = self.expert.index(None)
        self.expert[s], self.last[s] = e, self.tick
        return True

    def replace(self, e, protect):
        if e in self.expert:
            return False
        cands = [(self.last[s], x, s) for s, x in enumerate(self.expert) if x is not None and x not in protect]
        if not cands:
            return False
        _, _, s = min(cands)
        self.expert[s], self.last[s] = e, self.tick
        return True

    def prefetch(self, predicted, max_swaps):
        loads = swaps = 0
        for e in predicted:
            if self.admit(e):
                loads += 1
            elif swaps < max_swaps and self.replace(e, predicted):
                swaps += 1
        return loads, swaps


@pytest.mark.parametrize("fused,rows", [(True, 1), (False, 1), (True, 3)])
def test_lookahead_loads_the_next_layers_prediction(gpu, fused, rows):
    """Layer 1's experts are predicted from layer 0's activation with layer 1's
    router (its logits, bias included), merged by votes, loaded into empty slots or swapped
    over LRU residents (lookahead_swaps * rows at most), and layer 1's next
    step reads them as hits after waiting for the claim; its output stays
    within the bar of the oracle."""
    nm = gpu
    E, H, I, k, swaps_per_row = 16, 256, 256, 4, 2
    usable1 = 6
    copy, stream = nm.Stream(), nm.Stream()
    ring = nm.policy.StagingRing()
    l0, _, _, host0 = make_layer(nm, 1500, E, H, I, k, E, ring, copy)
    l1, banks1, stacks1, host1 = make_layer(nm, 1501, E, H, I, k, usable1, ring, copy, bias_scale=0.5)
    for e in range(E):
        assert l0.fill(e) == e
    model = SlotModel(usable1)
    out0, out1 = nm.DeviceBuffer(rows * H * 4), nm.DeviceBuffer(rows * H * 4)
    nm.policy.stats(reset=True)
    loads = swaps = 0
    for step in range(6):
        print(f"[lookahead fused={fused} rows={rows} step {step}]", flush=True)
        x = S.activations_bf16(1600 + step, rows, H)
        xd = nm.DeviceBuffer.from_array(x)
        if fused:
            info0, ahead = l0.forward_ahead(l1, xd, rows, out0, lookahead_swaps=swaps_per_row, promote_cap=0,
                                            stream=stream.handle)
            assert info0["hits"] == rows * k
        else:
            ahead = l1.prefetch_predicted(xd, rows, lookahead_swaps=swaps_per_row, stream=stream.handle)
        g, u, d, r, bias, dt, _ = host1
        logits = (O.router_logits(O.from_bf16(x), r) + bias).astype(np.float32)
        want_pred = nm.policy.union_by_votes([nm.policy.top_k_ids(row, k) for row in logits])
        assert l1.predicted() == want_pred
        resident = sum(model.resident(e) for e in want_pred)
        want_loads, want_swaps = model.prefetch(want_pred, swaps_per_row * rows)
        assert (ahead["predicted"], ahead["resident"], ahead["loads"], ahead["swaps"]) == \
            (len(want_pred), resident, want_loads, want_swaps), (step, ahead)
        assert ahead["pcie_bytes"] == (want_loads + want_swaps) * sum(stacks1.expert_bytes)
        loads, swaps = loads + want_loads, swaps + want_swaps
        # layer 1 runs on the same activation: its routing is the prediction
        info1 = l1.forward(xd, rows, out1, pcie_frac=1.0, promote_cap=0, stream=stream.handle)
        stream.sync()
        ids, _ = l1.routing(rows)
        assert info1["hits"] == model.route(ids.reshape(-1).tolist())
        assert info1["preload_waits"] == 1
        want_ids, _, want = oracle_step(host1, x, E, k, H)
        assert np.array_equal(ids, want_ids)
        err = S.max_rel_err(out1.download(np.float32).reshape(rows, H), want)
        print(f"  ahead={ahead} hits={info1['hits']} err={err:.3e}", flush=True)
        assert err < TOL
        if fused:
            _, _, want0 = oracle_step(host0, x, E, k, H)
            assert S.max_rel_err(out0.download(np.float32).reshape(rows, H), want0) < TOL
    assert swaps > 0 and loads == usable1
    st = nm.policy.stats()
    assert st["lookahead_loads"] == loads and st["swaps"] == swaps
    # the slots hold the experts the policy says, byte for byte
    table = l1.cache.slot_table()
    assert sorted(int(e) for e in np.nonzero(table >= 0)[0]) == sorted(model.expert)
    for e in np.nonzero(table >= 0)[0]:
        s = int(table[e])
        for proj, bank in enumerate((banks1.gate, banks1.up, banks1.down)):
            got = bank.buffer.download(np.uint8, count=bank.expert_bytes, offset=bank.offset + s * bank.stride)
            assert np.array_equal(got, stacks1.view(proj)[e]), (e, s, proj)


def test_profile_seeds_the_cache(gpu, tmp_path):
    """Seeding from an expert profile (src/moe/provider.rs:214-256): each layer
    takes the first round(usable * fill_share) experts of its ranking in order,
    a resident or out-of-model expert using its place; the seeded slots hold the
    experts' bytes and a step over them matches the oracle."""
    nm = gpu
    from naiwa_moe.policy import ExpertProfile, write_profile
    E, H, I, k, usable, rows = 16, 256, 256, 4, 6, 1
    ranking = [5, 9, 5, 20, 3, 1, 14, 8, 2]
    path = tmp_path / "profile.bin"
    write_profile(path, [(0, e) for e in ranking] + [(1, 7)], 2, 32)
    prof = ExpertProfile(path)
    assert prof.layer(0) == [5, 9, 20, 3, 1, 14, 8, 2]
    copy, stream = nm.Stream(), nm.Stream()
    ring = nm.policy.StagingRing()
    layer, banks, stacks, host = make_layer(nm, 1700, E, H, I, k, usable, ring, copy)
    assert layer.fill(3) == 0
    print("[profile] seeding", flush=True)
    assert layer.seed(prof.layer(0)) == 4   # 5, 9, 1, 14 (20: not in the model, 3: resident)
    table = layer.cache.slot_table()
    assert {e: int(table[e]) for e in np.nonzero(table >= 0)[0]} == {3: 0, 5: 1, 9: 2, 1: 3, 14: 4}
    for e, s in ((5, 1), (9, 2), (1, 3), (14, 4)):
        for proj, bank in enumerate((banks.gate, banks.up, banks.down)):
            got = bank.buffer.download(np.uint8, count=bank.expert_bytes, offset=bank.offset + s * bank.stride)
            assert np.array_equal(got, stacks.view(proj)[e]), (e, s, proj)
    out = nm.DeviceBuffer(rows * H * 4)
    x = S.activations_bf16(1701, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    layer.forward(xd, rows, out, pcie_frac=1.0, promote_cap=0, stream=stream.handle)
    stream.sync()
    _, _, want = oracle_step(host, x, E, k, H)
    assert S.max_rel_err(out.download(np.float32).reshape(rows, H), want) < TOL
    # half the slots: the first 3 of the ranking (20 is skipped, so 2 placed)
    layer2, _, _, _ = make_layer(nm, 1702, E, H, I, k, usable, ring, copy)
    assert layer2.seed(prof.layer(0), fill_share=0.5) == 2
    t2 = layer2.cache.slot_table()
    assert int(t2[5]) == 0 and int(t2[9]) == 1 and int((t2 >= 0).sum()) == 2


class PageableStacks:
    """Host expert stacks in ordinary pageable memory (e.g. a GGUF file read into
    a buffer): no device mapping, so staged uploads take one DMA copy per
    projection instead of the batched copy kernel."""

    def __init__(self, experts, hidden, inter, dtypes):
        from types import SimpleNamespace
        shapes = ((inter, hidden, dtypes[0]), (inter, hidden, dtypes[1]), (hidden, inter, dtypes[2]))
        self.expert_bytes = [n * O.row_bytes(dt, k) for n, k, dt in shapes]
        self.arrays = [np.zeros((experts, b), dtype=np.uint8) for b in self.expert_bytes]
        self.buffers = [SimpleNamespace(ptr=a.ctypes.data) for a in self.arrays]

    def view(self, proj):
        return self.arrays[proj]


@pytest.mark.parametrize("sync", ["event", "poll"])
@pytest.mark.parametrize("host_mem", ["pinned", "pageable", "contiguous"])
def test_cached_layer_alternating_streams(gpu, host_mem, sync):
    """Steps alternate between two compute streams with no host synchronisation of
    their own: a staged upload into a ring slot must come after every earlier read of
    that slot -- the expert kernel's and the promotion copy's -- which the step order
    guarantees (a step's routing waits for the previous step's last read, and the
    host queues the uploads only after that routing).  Every step's output matches
    the oracle and every resident (promoted) expert's three projections hold its
    bytes.  With pageable host stacks the uploads are per-projection DMA copies."""
    nm = gpu
    E, H, I, k, usable, rows = 16, 256, 256, 4, 4, 1
    copy = nm.Stream()
    streams = [nm.Stream(), nm.Stream()]
    ring = nm.policy.StagingRing()
    dt = (O.Q4_K,) * 3
    g, u, d, r = S.layer(1800, E, H, I, dt)
    if host_mem == "pageable":
        stacks = PageableStacks(E, H, I, dt)
    else:
        stacks = nm.HostExpertStacks(E, H, I, dt, interleaved=host_mem == "contiguous")
    for p_, src in enumerate((g, u, d)):
        stacks.view(p_)[:] = src.reshape(E, -1)
    banks = nm.LayerBanks(usable + ring.length, H, I, dt, contiguous=host_mem == "contiguous")
    router = nm.DeviceBuffer.from_array(r)
    bias = zipf_bias(E, 1.1, 1800)
    bias_d = nm.DeviceBuffer.from_array(bias)
    layer = nm.policy.CachedLayer(router, banks, stacks, E, k, usable, ring, copy.handle,
                                  mode=O.ROUTE_SOFTMAX_TOPK_RENORM, router_bias=bias_d)
    layer.set_upload_sync(nm.policy.UPLOAD_SYNC_POLL if sync == "poll" else nm.policy.UPLOAD_SYNC_EVENT)
    host = (g, u, d, r, bias, dt, I)
    steps = 10
    xs = [S.activations_bf16(1810 + i, rows, H) for i in range(steps)]
    xds = [nm.DeviceBuffer.from_array(x) for x in xs]
    outs = [nm.DeviceBuffer(rows * H * 4) for _ in range(steps)]
    promoted = 0
    for i in range(steps):
        print(f"[alternating streams {host_mem} {sync} step {i}]", flush=True)
        info = layer.forward(xds[i], rows, outs[i], pcie_frac=1.0, promote_cap=1, min_hits=1,
                             stream=streams[i % 2].handle)
        promoted += info["promoted"]
    for st in streams:
        st.sync()
    copy.sync()
    for i in range(steps):
        _, _, want = oracle_step(host, xs[i], E, k, H)
        err = S.max_rel_err(outs[i].download(np.float32).reshape(rows, H), want)
        assert err < TOL, (i, err)
    assert promoted > 0
    assert layer.upload_timeouts() == 0
    check_resident_bytes(layer, banks, stacks)


class PromotingSlotModel(SlotModel):
    """SlotModel plus the reference's promotion (src/moe/cached_layer.rs:892-1051):
    the step's staged experts in id order, at most cap of them; an expert already
    resident or seen fewer than min_hits times is skipped; the target is the first
    empty usable slot, else the slot with the smallest (last_use, slot) among those
    this step did not read (last_use < tick); a promoted slot is published with
    last_use = tick."""

    def __init__(self, usable, E):
        super().__init__(usable)
        self.hits = [0] * E

    def route(self, ids):
        for e in ids:
            self.hits[e] += 1
        return super().route(ids)

    def promote(self, staged, cap, min_hits):
        done = []
        for e in sorted(set(staged)):
            if len(done) >= cap:
                break
            if e in self.expert or self.hits[e] < min_hits:
                continue
            if None in self.expert:
                s = self.expert.index(None)
            else:
                cands = [(self.last[s], s) for s in range(len(self.expert)) if self.last[s] < self.tick]
                if not cands:
                    continue
                s = min(cands)[1]
            self.expert[s], self.last[s] = e, self.tick
            done.append(e)
        return done


def streamed(flat_ids, flat_w, resident, frac, cap):
    """The reference's streamed_misses (src/moe/cached_layer.rs:381-398), restated: the
    missed ids in order of first appearance with their weights summed in row-major
    order in f32, take = min(ceil(frac * distinct), cap), ranked by (sum desc, id asc)."""
    order, sums = [], {}
    for e, w in zip(flat_ids, flat_w):
        if resident(e):
            continue
        if e not in sums:
            order.append(e)
            sums[e] = np.float32(0.0)
        sums[e] = np.float32(sums[e] + np.float32(w))
    if not frac > 0:
        return []
    take = min(int(np.ceil(np.float32(frac) * np.float32(len(order)))), cap)
    return sorted(order, key=lambda e: (-float(sums[e]), e))[:take]


@pytest.mark.parametrize("sync,frac", [("event", 1.0), ("poll", 1.0), ("event", 0.5), ("event", 0.0)])
def test_cached_qwen3_shape_zipf(gpu, sync, frac):
    """The 25 %-cache workload at its real shape: two chained Qwen3-30B-A3B-shaped
    layers (H 2048, 128 experts, top-8, I 768, Q4_K), 32 cached experts + the
    16-slot staging ring per layer, Zipf(1.1) routing bias, the caches seeded with
    each layer's 32 most popular experts, 12 decode steps with staging of the
    pcie_frac share of the misses and one promotion per layer per step (min_hits 2);
    the other misses run on the CPU (pcie_frac 0: all of them, the reference's
    default).  Staged uploads complete through an event or the polled flag.  Every
    step: top-k ids bit-exact with the oracle on the GPU's own x_l, hit / staged /
    CPU counts and the slot table equal to an independent replay of the reference's
    policy, and the layer's output within 1e-2 of the oracle.  At the end every
    resident expert's three projections hold its bytes."""
    nm = gpu
    L, E, H, I, k, usable, rows, steps, min_hits = 2, 128, 2048, 768, 8, 32, 1, 12, 2
    dt = (O.Q4_K,) * 3
    copy, stream = nm.Stream(), nm.Stream()
    ring = nm.policy.StagingRing()
    proj = [nm.row_bytes(dt[0], H) * I, nm.row_bytes(dt[1], H) * I, nm.row_bytes(dt[2], I) * H]
    tmp = nm.DeviceBuffer(E * max(proj))
    layers, models, hosts, keep = [], [], [], []
    for l in range(L):
        # the benchmark's layout: each expert's projections adjacent on the host and in its slot
        stacks = nm.HostExpertStacks(E, H, I, dt, interleaved=True)
        for t in range(3):
            n, kk = (I, H) if t < 2 else (H, I)
            nm.synth(dt[t], 2000 + 8 * l + t, E * n * kk, tmp, 0.0, 0.02, stream=stream.handle)
            assert nm.lib().naiwa_memcpy_2d(stacks.ptrs[t], stacks.stride, tmp.ptr, proj[t], proj[t], E,
                                            stream.handle) == 0
            stream.sync()
        r = O.normal(S.stream(2000 + l, S.T_ROUTER), E * H, 0.0, 0.02).reshape(E, H)
        bias = zipf_bias(E, 1.1, 2100 + l)
        router, bias_d = nm.DeviceBuffer.from_array(r), nm.DeviceBuffer.from_array(bias)
        banks = nm.LayerBanks(usable + ring.length, H, I, dt, contiguous=True)
        layer = nm.policy.CachedLayer(router, banks, stacks, E, k, usable, ring, copy.handle,
                                      mode=O.ROUTE_SOFTMAX_TOPK_RENORM, router_bias=bias_d)
        layer.set_upload_sync(nm.policy.UPLOAD_SYNC_POLL if sync == "poll" else nm.policy.UPLOAD_SYNC_EVENT)
        # the 32 most popular experts (largest bias) first; at pcie_frac 0.5 only 12, so
        # that steps miss several experts and split them between the ring and the CPU
        seeded = usable if frac != 0.5 else 12
        popular = [int(e) for e in np.argsort(-bias, kind="stable")[:seeded]]
        assert layer.seed(popular) == seeded
        model = PromotingSlotModel(usable, E)
        for e in popular:
            model.admit(e)
        g, u, d = (np.ascontiguousarray(stacks.view(t)).reshape(E, *((I, -1) if t < 2 else (H, -1)))
                   for t in range(3))
        hosts.append((g, u, d, r, bias, dt, I))
        layers.append((layer, banks, stacks))
        models.append(model)
        keep += [router, bias_d]
    x = S.activations_bf16(2200, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    out = nm.DeviceBuffer(rows * H * 4)
    tot = {"staged": 0, "promoted": 0, "cpu": 0}
    both_in_one_step = False
    for step in range(steps):
        for l, (layer, banks, stacks) in enumerate(layers):
            print(f"[cached qwen3 {sync} frac={frac} step {step} layer {l}]", flush=True)
            info = layer.forward(xd, rows, out, pcie_frac=frac, promote_cap=1, min_hits=min_hits,
                                 stream=stream.handle)
            stream.sync()
            ids, w = layer.routing(rows)
            want_ids, want_w, want = oracle_step(hosts[l], x, E, k, H)
            assert np.array_equal(ids, want_ids), (step, l, ids, want_ids)
            assert np.allclose(w, want_w, rtol=1e-5, atol=1e-7)
            flat, flat_w = ids.reshape(-1).tolist(), w.reshape(-1).tolist()
            model = models[l]
            chosen = streamed(flat, flat_w, model.resident, frac, ring.length)
            staged = sorted(chosen)
            n_staged = sum(1 for e in flat if e in chosen and not model.resident(e))
            n_cpu = sum(1 for e in flat if not model.resident(e) and e not in chosen)
            hits = model.route(flat)
            assert info["hits"] == hits and info["staged_experts"] == len(staged), (step, l, info)
            assert info["staged"] == n_staged and info["cpu"] == n_cpu, (step, l, info)
            promoted = model.promote(staged, 1, min_hits)
            assert info["promoted"] == len(promoted), (step, l, info, promoted)
            table = layer.cache.slot_table()
            want_table = np.full(E, -1, dtype=np.int64)
            for s_, e in enumerate(model.expert):
                if e is not None:
                    want_table[e] = s_
            assert np.array_equal(table, want_table), (step, l)
            y = out.download(np.float32).reshape(rows, H)
            err = S.max_rel_err(y, want)
            print(f"  hits={info['hits']} staged={info['staged_experts']} promoted={info['promoted']} "
                  f"err={err:.3e}", flush=True)
            assert err < TOL, (step, l, err)
            tot["staged"] += info["staged_experts"]
            tot["promoted"] += info["promoted"]
            tot["cpu"] += info["cpu"]
            both_in_one_step |= info["staged_experts"] > 0 and info["cpu"] > 0
            x = O.to_bf16(O.from_bf16(x).astype(np.float32) + y)
            xd = nm.DeviceBuffer.from_array(x)
        # the next step starts from a fresh token
        x = S.activations_bf16(2201 + step, rows, H)
        xd = nm.DeviceBuffer.from_array(x)
    assert (tot["staged"] > 0 and tot["promoted"] > 0) == (frac > 0), tot
    assert (tot["cpu"] > 0) == (frac < 1), tot
    if frac == 0.5:
        assert both_in_one_step, "no step split its misses between the ring and the CPU"
    for layer, banks, stacks in layers:
        assert layer.upload_timeouts() == 0
        check_resident_bytes(layer, banks, stacks)


@pytest.mark.parametrize("swaps", [-1, 2])
def test_cached_stack_forward_matches_the_layer_calls(gpu, swaps):
    """naiwa_cached_stack_forward runs each layer's step and residual in order: the
    same routing, staging, promotions, lookahead and x bits as calling every layer's
    forward (or forward_ahead) and the residual add one by one."""
    nm = gpu
    E, H, I, k, usable, rows, L, steps = 16, 256, 256, 4, 4, 2, 3, 4
    stream = nm.Stream()
    runs = []
    for driver in ("layers", "stack"):
        copy = nm.Stream()
        ring = nm.policy.StagingRing()
        built = [make_layer(nm, 1500 + l, E, H, I, k, usable, ring, copy) for l in range(L)]
        layers = [b[0] for b in built]
        for layer in layers:
            layer.seed(list(range(usable)))
        x = nm.DeviceBuffer.from_array(S.activations_bf16(1510, rows, H))
        y = nm.DeviceBuffer(rows * H * 4)
        reports = []
        for _ in range(steps):
            if driver == "stack":
                info, ahead = nm.policy.CachedLayer.stack_forward(layers, x, rows, y, lookahead_swaps=swaps,
                                                                  stream=stream.handle)
            else:
                info = {"hits": 0, "staged": 0, "staged_experts": 0, "promoted": 0, "pcie_bytes": 0, "cpu": 0,
                        "preload_waits": 0}
                ahead = {"predicted": 0, "resident": 0, "loads": 0, "swaps": 0, "pcie_bytes": 0}
                for l, layer in enumerate(layers):
                    if swaps >= 0 and l + 1 < L:
                        s, a = layer.forward_ahead(layers[l + 1], x, rows, y, lookahead_swaps=swaps,
                                                   stream=stream.handle)
                        for f in ahead:
                            ahead[f] += a[f]
                    else:
                        s = layer.forward(x, rows, y, stream=stream.handle)
                    for f in info:
                        info[f] += s[f]
                    nm._lib.check(nm.lib().naiwa_residual_add_bf16(x.ptr, y.ptr, rows * H, stream.handle),
                                  "residual")
            reports.append((info, ahead if swaps >= 0 else None))
        stream.sync()
        runs.append((x.download(np.uint16), reports, [layer.cache.slot_table().tolist() for layer in layers]))
        del built, layers
    (xa, ra, sa), (xb, rb, sb) = runs
    assert ra == rb
    assert sa == sb
    assert np.array_equal(xa, xb)
    assert any(r[0]["staged"] for r in ra)   # the run stages misses


def _policy_state(layer, ring):
    c = layer.cache
    return (c.tick, c.hit_counts().tolist(), [c.slot_state(s) for s in range(c.slots)], ring.acquire(0))


def test_cpu_misses_off_refuses_the_step_before_any_state_changes(gpu):
    """With the CPU path switched off, a step whose misses the ring does not take
    (pcie_frac 0) is refused with NAIWA_E_UNSUPPORTED, and the tick, the hit counts,
    every slot's state and the ring cursor are as before.  Switched on again, the same
    step runs its misses on the CPU and matches the oracle."""
    nm = gpu
    E, H, I, k, usable, rows = 16, 256, 256, 4, 4, 2
    copy, stream = nm.Stream(), nm.Stream()
    ring = nm.policy.StagingRing()
    layer, banks, stacks, host = make_layer(nm, 2600, E, H, I, k, usable, ring, copy)
    for e in range(usable):
        assert layer.fill(e) == e
    x = S.activations_bf16(2601, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    out = nm.DeviceBuffer(rows * H * 4)
    layer.set_cpu_misses(False)
    before = _policy_state(layer, ring)
    with pytest.raises(nm.NaiwaError) as e:
        layer.forward(xd, rows, out, pcie_frac=0.0, stream=stream.handle)
    assert e.value.rc == nm.E_UNSUPPORTED
    assert _policy_state(layer, ring) == before
    layer.set_cpu_misses(True)
    info = layer.forward(xd, rows, out, pcie_frac=0.0, stream=stream.handle)
    stream.sync()
    assert info["cpu"] > 0 and info["staged_experts"] == 0 and info["hits"] + info["cpu"] == rows * k
    _, _, want = oracle_step(host, x, E, k, H)
    assert S.max_rel_err(out.download(np.float32).reshape(rows, H), want) < TOL


def test_poll_upload_wait_that_runs_out_is_reported_by_the_next_step(gpu):
    """Poll mode with the device wait bound forced to 1 us from the host and the copy
    stream kept busy, so the staged-upload wait of a step gives up: the wait counts it
    in the layer's doorbell, and the layer's next forward returns NAIWA_E_TIMEOUT before
    it changes any policy state.  With the bound restored the layer goes on and its
    outputs match the oracle again."""
    nm = gpu
    L = nm.lib()
    E, H, I, k, usable, rows = 16, 256, 256, 4, 2, 1
    copy, stream = nm.Stream(), nm.Stream()
    ring = nm.policy.StagingRing()
    layer, banks, stacks, host = make_layer(nm, 2700, E, H, I, k, usable, ring, copy)
    layer.set_upload_sync(nm.policy.UPLOAD_SYNC_POLL)
    x = S.activations_bf16(2701, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    out = nm.DeviceBuffer(rows * H * 4)
    big_src, big_dst = nm.DeviceBuffer(256 << 20), nm.DeviceBuffer(256 << 20)
    assert L.naiwa_memcpy_d2d(big_dst.ptr, big_src.ptr, 256 << 20, copy.handle) == 0   # the copy stream is busy
    L.naiwa_doorbell_set_wait_limit_us(1)
    try:
        info = layer.forward(xd, rows, out, pcie_frac=1.0, stream=stream.handle)   # nothing cached: all staged
        stream.sync()
    finally:
        L.naiwa_doorbell_set_wait_limit_us(0)
    copy.sync()
    assert info["staged_experts"] > 0
    assert layer.upload_timeouts() == 1
    before = _policy_state(layer, ring)
    with pytest.raises(nm.NaiwaError) as e:
        layer.forward(xd, rows, out, pcie_frac=1.0, stream=stream.handle)
    assert e.value.rc == nm.E_TIMEOUT
    assert _policy_state(layer, ring) == before
    info = layer.forward(xd, rows, out, pcie_frac=1.0, stream=stream.handle)
    stream.sync()
    _, _, want = oracle_step(host, x, E, k, H)
    assert S.max_rel_err(out.download(np.float32).reshape(rows, H), want) < TOL
    assert layer.upload_timeouts() == 1


@pytest.mark.parametrize("rows", [2, 5])
def test_upload_waits_and_paths_give_the_same_bits(gpu, rows):
    """Identical layers whose staged uploads travel as one copy kernel or as DMA
    copies, and complete into the expert pass through the polled device flag or an
    event, run the same ten steps (pcie_frac 1 and 0.5 alternating, so some steps also
    run misses on the CPU): the outputs are identical bit for bit, as are the per-step
    counts, and they match the oracle.  At 2 rows the poll wait rides in the gate/up
    blocks; at 5 rows (the matrix-core pass) one wave waits before the pass."""
    nm = gpu
    E, H, I, k, usable = 16, 256, 256, 4, 4
    outs = {}
    for sync, path in (("event", "kernel"), ("poll", "kernel"), ("poll", "dma"), ("event", "dma")):
        copy, stream = nm.Stream(), nm.Stream()
        ring = nm.policy.StagingRing()
        layer, banks, stacks, host = make_layer(nm, 2800, E, H, I, k, usable, ring, copy)
        layer.set_upload_sync(nm.policy.UPLOAD_SYNC_POLL if sync == "poll" else nm.policy.UPLOAD_SYNC_EVENT)
        layer.set_upload_path(nm.policy.UPLOAD_PATH_DMA if path == "dma" else nm.policy.UPLOAD_PATH_KERNEL)
        res = []
        for i in range(10):
            print(f"[{sync} {path} rows {rows} step {i}]", flush=True)
            x = S.activations_bf16(2810 + i, rows, H)
            out = nm.DeviceBuffer(rows * H * 4)
            info = layer.forward(nm.DeviceBuffer.from_array(x), rows, out, pcie_frac=1.0 if i % 2 == 0 else 0.5,
                                 promote_cap=1, min_hits=1, stream=stream.handle)
            stream.sync()
            y = out.download(np.float32).reshape(rows, H)
            _, _, want = oracle_step(host, x, E, k, H)
            assert S.max_rel_err(y, want) < TOL, (sync, i)
            res.append((y, info["hits"], info["staged_experts"], info["cpu"]))
        copy.sync()
        assert layer.upload_timeouts() == 0
        outs[(sync, path)] = res
    first = outs[("event", "kernel")]
    for key, res in outs.items():
        for (ye, *ce), (yp, *cp) in zip(first, res):
            assert np.array_equal(ye.view(np.uint32), yp.view(np.uint32)), key
            assert ce == cp, key
    assert sum(r[3] for r in first) > 0 and sum(r[2] for r in first) > 0


def test_lookahead_into_a_layer_of_another_top_k_is_refused(gpu):
    """forward_ahead publishes the next layer's prediction in this layer's top_k
    columns, so a next layer with another top_k is refused with NAIWA_E_INVALID
    before any state changes; the same layer still runs a plain forward after it."""
    nm = gpu
    E, H, I, usable, rows = 16, 256, 256, 4, 1
    copy, stream = nm.Stream(), nm.Stream()
    ring0, ring1 = nm.policy.StagingRing(), nm.policy.StagingRing()
    l0, banks0, stacks0, host0 = make_layer(nm, 2900, E, H, I, 4, usable, ring0, copy)
    l1, banks1, stacks1, host1 = make_layer(nm, 2910, E, H, I, 2, usable, ring1, copy)
    x = S.activations_bf16(2901, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    out = nm.DeviceBuffer(rows * H * 4)
    before = _policy_state(l0, ring0)
    with pytest.raises(nm.NaiwaError) as e:
        l0.forward_ahead(l1, xd, rows, out, lookahead_swaps=2, stream=stream.handle)
    assert e.value.rc == nm.E_INVALID
    assert _policy_state(l0, ring0) == before
    l0.forward(xd, rows, out, pcie_frac=1.0, stream=stream.handle)
    stream.sync()
    _, _, want = oracle_step(host0, x, E, 4, H)
    assert S.max_rel_err(out.download(np.float32).reshape(rows, H), want) < TOL
