"""GPU parity of the partial-cache decode step (include/naiwa_cached.h): device
routing with a per-expert bias is bit-exact with the oracle, the hit/miss split
and staging follow the host policy, staged experts are uploaded byte-exactly into
their ring slots, promotion moves them into the cache, and every step's expert
output is within the 1e-2 relative bar of the oracle over the same routed set."""
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
    # promoted experts are resident and their bytes are the expert's bytes
    table = layer.cache.slot_table()
    for e in np.nonzero(table >= 0)[0]:
        s = int(table[e])
        got = banks.gate.buffer.download(np.uint8, count=banks.gate.expert_bytes, offset=s * banks.gate.stride)
        assert np.array_equal(got, stacks.view(0)[e]), (e, s)


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
            got = bank.buffer.download(np.uint8, count=bank.expert_bytes, offset=(usable + pos) * bank.stride)
            assert np.array_equal(got, stacks.view(proj)[e])
