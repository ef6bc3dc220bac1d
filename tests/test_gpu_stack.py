"""GPU parity of naiwa_stack_decode (fused persistent kernel and the layered
chain) against the oracle, layer by layer with teacher forcing: for every layer
the router top-k computed from the GPU's own input x_l is bit-exact, and the
layer's expert output is within the 1e-2 relative bar."""
import numpy as np
import pytest

import oracle as O
import synthetic as S

pytestmark = pytest.mark.gpu
TOL = 1e-2


def build_stack(nm, L, H, E, I, dt, seed, slots_perm=False, tie_pairs=False):
    layers, host, keep = [], [], []
    for l in range(L):
        g, u, d, r = S.layer(seed + l, E, H, I, dt)
        if tie_pairs:
            # experts 2j and 2j + 1 share a router row: their logits are equal
            r = r.copy()
            r[1::2] = r[0::2]
        banks = nm.LayerBanks(E + (3 if slots_perm else 0), H, I, dt)
        slot_of = np.arange(E, dtype=np.int32)
        if slots_perm:
            slot_of = ((np.arange(E) * 5 + 3) % (E + 3)).astype(np.int32)
        for e in range(E):
            banks.load(int(slot_of[e]), g[e], u[e], d[e])
        rd = nm.DeviceBuffer.from_array(r)
        table = nm.DeviceBuffer.from_array(slot_of) if slots_perm else None
        layers.append(nm.layer_desc(rd, banks, table))
        keep += [banks, rd, table]
        host.append((r, (g, u, d), dt, I))
    return layers, host, keep


def oracle_layer(host_layer, x_bf16, E, k, mode, H):
    r, (g, u, d), dt, I = host_layer
    xf = O.from_bf16(x_bf16)
    ids, w = O.topk(O.router_logits(xf, r), k, mode)
    gs, us, ds = O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I)
    y = O.fused_moe_decode(gs, us, ds, xf, ids, w)
    return ids, w, y


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("rows,L,H,E,k,I,dt,mode,perm", [
    (1, 3, 2048, 128, 8, 768, (O.Q4_K,) * 3, O.ROUTE_SOFTMAX_TOPK_RENORM, False),  # Qwen3 shape
    (1, 2, 1024, 8, 2, 2048, (O.Q8_0,) * 3, O.ROUTE_TOPK_SOFTMAX, True),
    (1, 2, 2048, 64, 6, 1408, (O.Q4_K, O.Q4_K, O.Q8_0), O.ROUTE_SOFTMAX_TOPK, True),
    (1, 2, 512, 256, 8, 256, (O.Q8_0,) * 3, O.ROUTE_SOFTMAX_TOPK_RENORM, True),   # 256 experts
    (8, 2, 2048, 128, 8, 768, (O.Q4_K,) * 3, O.ROUTE_SOFTMAX_TOPK_RENORM, True),
    (3, 2, 1024, 8, 2, 2048, (O.Q8_0,) * 3, O.ROUTE_TOPK_SOFTMAX, False),          # C1 shape
    (2, 2, 2048, 64, 6, 1408, (O.Q4_K, O.Q4_K, O.Q8_0), O.ROUTE_SOFTMAX_TOPK, True),  # DS-V2-Lite
])
def test_stack_layer_by_layer(gpu, fused, rows, L, H, E, k, I, dt, mode, perm):
    nm = gpu
    layers, host, keep = build_stack(nm, L, H, E, I, dt, 900 + rows, slots_perm=perm)
    x = S.activations_bf16(901 + rows, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    ids_d = nm.DeviceBuffer(rows * k * 4)
    w_d = nm.DeviceBuffer(rows * k * 4)
    for l in range(L):
        print(f"[stack fused={fused} rows={rows} H={H} E={E} layer={l}]", flush=True)
        x_in = xd.download(np.uint16).reshape(rows, H)
        nm.stack_decode([layers[l]], xd, rows, H, E, k, mode=mode, ids_out=ids_d, w_out=w_d,
                        fused=fused)
        nm.synchronize()
        if fused:
            assert nm.stack_status() == (0, 0)
        ids = ids_d.download(np.uint32).reshape(rows, k)
        w = w_d.download(np.float32).reshape(rows, k)
        want_ids, want_w, y = oracle_layer(host[l], x_in, E, k, mode, H)
        assert np.array_equal(ids, want_ids), (l, ids, want_ids)
        assert np.allclose(w, want_w, rtol=1e-5, atol=1e-7)
        x_out = O.from_bf16(xd.download(np.uint16).reshape(rows, H))
        got_y = x_out - O.from_bf16(x_in)
        # bf16 storage of x adds up to half an ulp of |x| per element on top of y's error
        slack = np.abs(O.from_bf16(x_in)).max() * 2.0 ** -8 / max(np.abs(y).max(), 1e-30)
        err = S.max_rel_err(got_y, y)
        print(f"  max_rel_err(y)={err:.3e} slack={slack:.3e}", flush=True)
        assert err < TOL + slack


def test_fused_multi_layer_matches_oracle_chain(gpu):
    """Four Qwen3-shaped layers in one fused launch: while the routing stays
    identical, the final x follows the oracle's residual chain."""
    nm = gpu
    rows, L, H, E, k, I = 1, 4, 2048, 128, 8, 768
    dt = (O.Q4_K,) * 3
    layers, host, keep = build_stack(nm, L, H, E, I, dt, 950)
    x = S.activations_bf16(951, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    ids_d = nm.DeviceBuffer(L * rows * k * 4)
    w_d = nm.DeviceBuffer(L * rows * k * 4)
    nm.stack_decode(layers, xd, rows, H, E, k, ids_out=ids_d, w_out=w_d, fused=True)
    nm.synchronize()
    assert nm.stack_status() == (0, 0)
    got = O.from_bf16(xd.download(np.uint16).reshape(rows, H))
    want_x, want_ids, _ = O.stack_decode(host, x, E, k)
    ids = ids_d.download(np.uint32).reshape(L, rows, k)
    assert np.array_equal(ids[0], want_ids[0])
    if np.array_equal(ids, want_ids):
        delta = got - O.from_bf16(x)
        want_delta = O.from_bf16(want_x) - O.from_bf16(x)
        # each layer's bf16 store may round the other way: one ulp of |x| per layer
        slack = L * np.abs(got).max() * 2.0 ** -7 / np.abs(want_delta).max()
        assert S.max_rel_err(delta, want_delta) < TOL + slack


def test_fused_is_deterministic(gpu):
    nm = gpu
    rows, L, H, E, k, I = 2, 3, 2048, 128, 8, 768
    layers, _, keep = build_stack(nm, L, H, E, I, (O.Q4_K,) * 3, 970)
    x = S.activations_bf16(971, rows, H)
    outs = []
    for _ in range(3):
        xd = nm.DeviceBuffer.from_array(x)
        nm.stack_decode(layers, xd, rows, H, E, k, fused=True)
        nm.synchronize()
        outs.append(xd.download(np.uint16))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("rows,mode", [(1, O.ROUTE_SOFTMAX_TOPK_RENORM), (1, O.ROUTE_SOFTMAX_TOPK),
                                       (2, O.ROUTE_TOPK_SOFTMAX)])
def test_fused_routing_ties_take_the_lower_id(gpu, rows, mode):
    """Router rows duplicated in pairs make every selected logit tie with its
    twin: the order is (logit desc, id asc), so ids and weights stay bit-exact
    with the oracle's selection."""
    nm = gpu
    H, E, k, I = 1024, 64, 8, 256
    dt = (O.Q8_0,) * 3
    layers, host, keep = build_stack(nm, 1, H, E, I, dt, 990 + rows, tie_pairs=True)
    x = S.activations_bf16(991 + rows, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    ids_d = nm.DeviceBuffer(rows * k * 4)
    w_d = nm.DeviceBuffer(rows * k * 4)
    print(f"[stack ties rows={rows} mode={mode}]", flush=True)
    nm.stack_decode(layers, xd, rows, H, E, k, mode=mode, ids_out=ids_d, w_out=w_d, fused=True)
    nm.synchronize()
    assert nm.stack_status() == (0, 0)
    ids = ids_d.download(np.uint32).reshape(rows, k)
    w = w_d.download(np.float32).reshape(rows, k)
    want_ids, want_w, y = oracle_layer(host[0], x, E, k, mode, H)
    # the twins come out adjacent, even id first
    assert np.all(want_ids[:, 0::2] % 2 == 0) and np.array_equal(want_ids[:, 1::2], want_ids[:, 0::2] + 1)
    assert np.array_equal(ids, want_ids), (ids, want_ids)
    assert np.allclose(w, want_w, rtol=1e-5, atol=1e-7)
    got_y = O.from_bf16(xd.download(np.uint16).reshape(rows, H)) - O.from_bf16(x)
    slack = np.abs(O.from_bf16(x)).max() * 2.0 ** -8 / max(np.abs(y).max(), 1e-30)
    assert S.max_rel_err(got_y, y) < TOL + slack
