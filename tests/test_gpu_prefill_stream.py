"""GPU: the whole-layer prefill stream (include/naiwa_prefill.h) runs a chunk's MoE
layers over expert stacks in pinned host memory through a ring of `depth`
device layer buffers.  Every layer's output equals the resident prefill over the
same bytes bit for bit, and the oracle within the 1e-2 bar; a second chunk
reuses the buffers (uploads after the last read of each buffer)."""
import numpy as np
import pytest

import oracle as O
import synthetic as S

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_stream_matches_resident_prefill_and_oracle(gpu, depth):
    nm = gpu
    from naiwa_moe.prefill import PrefillStream
    L, E, k, H, I, T = 4, 8, 2, 256, 256, 40
    dt = (O.Q4_K, O.Q4_K, O.Q8_0)
    layers, stacks = [], []
    for l in range(L):
        g, u, d, r = S.layer(1800 + l, E, H, I, dt)
        hs = nm.HostExpertStacks(E, H, I, dt)
        for p, src in enumerate((g, u, d)):
            hs.view(p)[:] = src.reshape(E, -1)
        layers.append((g, u, d, r))
        stacks.append(hs)
    copy, stream = nm.Stream(), nm.Stream()
    ps = PrefillStream(stacks, H, I, dt, depth, copy.handle)
    x = S.activations_bf16(1900, T, H)
    xd = nm.DeviceBuffer.from_array(x)
    routed = []
    for g, u, d, r in layers:
        ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k)
        routed.append((nm.DeviceBuffer.from_array(ids.astype(np.uint32)), nm.DeviceBuffer.from_array(w), ids, w))
    outs = [nm.DeviceBuffer(T * H * 4) for _ in range(L)]
    for chunk in range(2):
        print(f"[prefill stream depth={depth} chunk {chunk}]", flush=True)
        for l in range(L):
            ids_d, w_d, _, _ = routed[l]
            ps.forward(l, xd, ids_d, w_d, T, k, outs[l], stream=stream.handle)
        stream.sync()
        for l, (g, u, d, r) in enumerate(layers):
            got = outs[l].download(np.float32).reshape(T, H)
            banks = nm.LayerBanks(E, H, I, dt)
            for e in range(E):
                banks.load(e, g[e], u[e], d[e])
            ref = nm.DeviceBuffer(T * H * 4)
            ids_d, w_d, ids, w = routed[l]
            nm.moe_prefill(banks, xd, ids_d, w_d, T, k, ref)
            nm.synchronize()
            assert np.array_equal(got, ref.download(np.float32).reshape(T, H)), (depth, chunk, l)
            gs, us, ds = O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I)
            err = S.max_rel_err(got, O.fused_moe_decode(gs, us, ds, O.from_bf16(x), ids, w))
            assert err < TOL, (depth, chunk, l, err)
    st = ps.stats()
    per_layer = E * sum(stacks[0].expert_bytes)
    # the ring: a forward of layer l loads l .. l + depth - 1 into buffers (l % depth)
    # unless the buffer already holds that layer
    held, want = [-1] * depth, 0
    for _ in range(2):
        for l in range(L):
            for ll in range(l, min(L, l + depth)):
                if held[ll % depth] != ll:
                    held[ll % depth], want = ll, want + 1
    print(f"  stats={st} want uploads={want}", flush=True)
    assert st["forwards"] == 2 * L and st["uploads"] == want and st["upload_bytes"] == want * per_layer
