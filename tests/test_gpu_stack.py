"""GPU parity of naiwa_stack_decode (fused persistent kernel and the layered
chain) against the oracle, layer by layer with teacher forcing: each launch
returns every layer's f32 MoE output y_l; for every layer the router top-k the
oracle computes from the GPU's own input x_l is bit-exact with the GPU's, and
y_l is within the 1e-2 relative bar of the oracle's expert output."""
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


def run_and_check(nm, layers, host, x, rows, H, E, k, mode, fused, label):
    """One naiwa_stack_decode launch over every layer with the per-layer f32 MoE
    outputs y_l captured, then teacher forcing on the GPU's own trajectory: the
    host rebuilds x_{l+1} = bf16(f32(x_l) + y_l) (bit-exact with the final x the
    kernel stored), and for every layer the oracle routes the same x_l bits --
    top-k ids bit-exact, weights to f32 rounding -- and its expert output must
    be within the 1e-2 norm-relative bar of y_l, with no allowance for bf16
    storage.  Returns the per-layer errors and the routed ids [L, rows, k]."""
    L = len(layers)
    xd = nm.DeviceBuffer.from_array(x)
    ids_d = nm.DeviceBuffer(L * rows * k * 4)
    w_d = nm.DeviceBuffer(L * rows * k * 4)
    y_d = nm.DeviceBuffer(L * rows * H * 4)
    print(f"[{label} fused={fused} rows={rows} H={H} E={E} k={k} L={L}]", flush=True)
    nm.stack_decode(layers, xd, rows, H, E, k, mode=mode, ids_out=ids_d, w_out=w_d, fused=fused, y_out=y_d)
    nm.synchronize()
    if fused:
        assert nm.stack_status() == (0, 0)
    ids = ids_d.download(np.uint32).reshape(L, rows, k)
    w = w_d.download(np.float32).reshape(L, rows, k)
    ys = y_d.download(np.float32).reshape(L, rows, H)
    errs = check_chain(host, x, ids, w, ys, xd.download(np.uint16).reshape(rows, H), rows, H, E, k, mode)
    return errs, ids


def check_chain(host, x, ids, w, ys, x_final, rows, H, E, k, mode):
    """Teacher-forced check of one launch's outputs (see run_and_check)."""
    L = len(host)
    x_l = x.copy()
    errs = []
    for l in range(L):
        want_ids, want_w, want_y = oracle_layer(host[l], x_l, E, k, mode, H)
        assert np.array_equal(ids[l], want_ids), (l, ids[l], want_ids)
        assert np.allclose(w[l], want_w, rtol=1e-5, atol=1e-7), l
        err = S.max_rel_err(ys[l], want_y)
        errs.append(err)
        print(f"  layer {l}: max_rel_err(y)={err:.3e}", flush=True)
        assert err < TOL, (l, err)
        x_l = O.to_bf16(O.from_bf16(x_l).astype(np.float32) + ys[l])
    # the kernel's stored x is the chain of its own y outputs, bit for bit
    assert np.array_equal(x_final, x_l)
    return errs


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("rows,L,H,E,k,I,dt,mode,perm", [
    (1, 4, 2048, 128, 8, 768, (O.Q4_K,) * 3, O.ROUTE_SOFTMAX_TOPK_RENORM, False),  # Qwen3 shape
    (1, 2, 2048, 64, 4, 768, (O.Q4_K,) * 3, O.ROUTE_SOFTMAX_TOPK_RENORM, True),    # any shape, Q4_K
    (8, 3, 2048, 128, 8, 768, (O.Q4_K,) * 3, O.ROUTE_SOFTMAX_TOPK_RENORM, True),   # Qwen3 shape, bs8
    (2, 3, 2048, 128, 8, 768, (O.Q4_K,) * 3, O.ROUTE_SOFTMAX_TOPK_RENORM, True),   # Qwen3 shape, bs2
    (1, 2, 1024, 8, 2, 2048, (O.Q8_0,) * 3, O.ROUTE_TOPK_SOFTMAX, True),
    (1, 2, 2048, 64, 6, 1408, (O.Q4_K, O.Q4_K, O.Q8_0), O.ROUTE_SOFTMAX_TOPK, True),
    (1, 2, 512, 256, 8, 256, (O.Q8_0,) * 3, O.ROUTE_SOFTMAX_TOPK_RENORM, True),   # 256 experts
    (3, 2, 1024, 8, 2, 2048, (O.Q8_0,) * 3, O.ROUTE_TOPK_SOFTMAX, False),          # C1 shape
    (2, 2, 2048, 64, 6, 1408, (O.Q4_K, O.Q4_K, O.Q8_0), O.ROUTE_SOFTMAX_TOPK, True),  # DS-V2-Lite
])
def test_stack_teacher_forced(gpu, fused, rows, L, H, E, k, I, dt, mode, perm):
    nm = gpu
    layers, host, keep = build_stack(nm, L, H, E, I, dt, 900 + rows, slots_perm=perm)
    x = S.activations_bf16(901 + rows, rows, H)
    run_and_check(nm, layers, host, x, rows, H, E, k, mode, fused, "stack")


@pytest.mark.parametrize("rows", [1, 8])
def test_fused_matches_layered_bit_for_bit_routing(gpu, rows):
    """The fused kernel and the layered chain route the same 4-layer Qwen3-shaped
    stack identically (each layer's ids come from its own x_l, which both paths
    rebuild from their y outputs) and both stay within 1e-2 of the oracle."""
    nm = gpu
    H, E, k, I, L = 2048, 128, 8, 768, 4
    layers, host, keep = build_stack(nm, L, H, E, I, (O.Q4_K,) * 3, 950)
    x = S.activations_bf16(951, rows, H)
    for fused in (True, False):
        run_and_check(nm, layers, host, x, rows, H, E, k, O.ROUTE_SOFTMAX_TOPK_RENORM, fused, "chain")


def test_fused_trace_records_phases_and_leaves_the_bits_unchanged(gpu):
    """The phase trace (a separate instantiation at the Qwen3 shape, with its marks
    compiled in) records every workgroup's timestamps, in order within each layer's
    first phases, and the traced launch gives the same ids, weights and x bits as the
    untraced one."""
    import ctypes as C
    nm = gpu
    lib = nm.lib()
    rows, L, H, E, k, I = 1, 2, 2048, 128, 8, 768
    layers, host, keep = build_stack(nm, L, H, E, I, (O.Q4_K,) * 3, 990)
    x = S.activations_bf16(991, rows, H)
    outs = []
    for trace in (0, 1, 0):
        xd = nm.DeviceBuffer.from_array(x)
        ids_d, w_d = nm.DeviceBuffer(L * rows * k * 4), nm.DeviceBuffer(L * rows * k * 4)
        print(f"[trace={trace}]", flush=True)
        assert lib.naiwa_stack_trace_enable(trace) == 0
        try:
            nm.stack_decode(layers, xd, rows, H, E, k, ids_out=ids_d, w_out=w_d, fused=True)
            nm.synchronize()
        finally:
            lib.naiwa_stack_trace_enable(0)
        assert nm.stack_status() == (0, 0)
        outs.append((ids_d.download(np.uint32), w_d.download(np.uint32), xd.download(np.uint16)))
        if trace:
            slots = 24
            cap = 4096 * (L + 1) * slots
            buf = (C.c_uint64 * cap)()
            nl, nb = C.c_int(0), C.c_int(0)
            assert lib.naiwa_stack_trace_read(buf, cap, C.byref(nl), C.byref(nb)) == 0
            assert nl.value == L and nb.value >= 16
            t = np.frombuffer(buf, dtype=np.uint64)[: nb.value * (L + 1) * slots].reshape(nb.value, L + 1, slots)
            # every workgroup: x received (0) <= ranked (1) <= routed (2) <= gate/up rows landed (3)
            for l in range(L):
                m = t[:, l, :4].astype(np.int64)
                assert (m > 0).all(), l
                assert (np.diff(m, axis=1) >= 0).all(), l
    for o in outs[1:]:
        for a_, b_ in zip(outs[0], o):
            assert np.array_equal(a_, b_)


def test_two_token_steps_give_the_same_bits_with_and_without_outputs(gpu):
    """Two tokens at the Qwen3 shape (two one-token launches whose outputs are
    interleaved afterwards): the updated x, ids and weights are bit-identical whether
    the call asks for the per-layer outputs, for ids and weights only, or for nothing."""
    nm = gpu
    rows, L, H, E, k, I = 2, 3, 2048, 128, 8, 768
    layers, host, keep = build_stack(nm, L, H, E, I, (O.Q4_K,) * 3, 1010)
    x = S.activations_bf16(1011, rows, H)
    res = []
    for mode in ("all", "ids", "none"):
        xd = nm.DeviceBuffer.from_array(x)
        ids_d, w_d = nm.DeviceBuffer(L * rows * k * 4), nm.DeviceBuffer(L * rows * k * 4)
        y_d = nm.DeviceBuffer(L * rows * H * 4) if mode == "all" else None
        print(f"[two tokens, outputs={mode}]", flush=True)
        nm.stack_decode(layers, xd, rows, H, E, k, ids_out=None if mode == "none" else ids_d,
                        w_out=None if mode == "none" else w_d, fused=True, y_out=y_d)
        nm.synchronize()
        assert nm.stack_status() == (0, 0)
        res.append((xd.download(np.uint16), ids_d.download(np.uint32), w_d.download(np.uint32)))
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][0], res[2][0])
    assert np.array_equal(res[0][1], res[1][1]) and np.array_equal(res[0][2], res[1][2])
    # each token's row of the routing is its own: the two tokens route differently
    ids = res[0][1].reshape(L, rows, k)
    assert any(not np.array_equal(np.sort(ids[l, 0]), np.sort(ids[l, 1])) for l in range(L))


def test_fused_status_counts_add_up_across_launches(gpu):
    """Pairs routed to an expert that has no slot are counted as missing (and left out of
    the output).  Each launch starts its own counts from zero and folds its predecessor's
    into the running totals, so launches in a row add up to the sum of their counts, a
    status read returns them and clears them, and no wait times out -- also over 1,100
    launches in a row without a status read."""
    nm = gpu
    L, H, E, I, k, rows, gone = 2, 256, 16, 256, 4, 2, 5
    dt = (O.Q4_K,) * 3
    layers, keep = [], []
    for l in range(L):
        g, u, d, r = S.layer(3100 + l, E, H, I, dt)
        r = r.copy()
        r[gone] *= 3.0  # larger logits either way: expert `gone` is often in the top k
        banks = nm.LayerBanks(E, H, I, dt)
        slot_of = np.arange(E, dtype=np.int32)
        slot_of[gone] = -1
        for e in range(E):
            if e != gone:
                banks.load(e, g[e], u[e], d[e])
        rd, table = nm.DeviceBuffer.from_array(r), nm.DeviceBuffer.from_array(slot_of)
        layers.append(nm.layer_desc(rd, banks, table))
        keep += [banks, rd, table]
    nm.stack_status()  # earlier tests' counts
    counts = []
    for launch in range(4):
        x = S.activations_bf16(3110 + launch, rows, H)
        xd = nm.DeviceBuffer.from_array(x)
        ids_d, w_d = nm.DeviceBuffer(L * rows * k * 4), nm.DeviceBuffer(L * rows * k * 4)
        print(f"[status launch {launch}]", flush=True)
        nm.stack_decode(layers, xd, rows, H, E, k, ids_out=ids_d, w_out=w_d, fused=True)
        nm.synchronize()
        counts.append(int((ids_d.download(np.uint32) == gone).sum()))
        if launch == 2:
            assert nm.stack_status() == (0, sum(counts))
    assert nm.stack_status() == (0, counts[3])
    assert nm.stack_status() == (0, 0)
    assert sum(counts) > 0
    # past the ring: the same token again and again, its count known from the first launch
    x = S.activations_bf16(3110, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    ids_d, w_d = nm.DeviceBuffer(L * rows * k * 4), nm.DeviceBuffer(L * rows * k * 4)
    n = 1100
    print(f"[status over {n} launches]", flush=True)
    total = 0
    for launch in range(n):
        xd.upload(x)
        nm.stack_decode(layers, xd, rows, H, E, k, ids_out=ids_d, w_out=w_d, fused=True)
        if launch % 100 == 0:
            nm.synchronize()
        if launch == 0:
            nm.synchronize()
            per = int((ids_d.download(np.uint32) == gone).sum())
            assert per == counts[0]
        total += per
    nm.synchronize()
    assert nm.stack_status() == (0, total)


def test_fused_last_slot_of_exact_bank(gpu):
    """Routing forced onto the last slot of a bank sized exactly to its experts (no
    slot stride padding past the last slot): the fused kernel's LDS prefetch of the
    down rows and its gate/up row DMA stay inside the allocation and the output
    matches the oracle."""
    nm = gpu
    rows, L, H, E, k, I = 1, 2, 2048, 128, 8, 768
    dt = (O.Q4_K,) * 3
    layers, host, keep = build_stack(nm, L, H, E, I, dt, 960)
    for l in range(L):
        r = host[l][0].copy()
        # experts E-8 .. E-1 (the bank's last slots) get a large router response
        r[E - 8:] += 0.05
        host[l] = (r, host[l][1], host[l][2], host[l][3])
        nm.lib().naiwa_memcpy_h2d(layers[l].router, r.ctypes.data, r.nbytes, 0)
    nm.synchronize()
    x = np.abs(O.from_bf16(S.activations_bf16(961, rows, H))).astype(np.float32)
    x = O.to_bf16(x)
    _, ids = run_and_check(nm, layers, host, x, rows, H, E, k, O.ROUTE_SOFTMAX_TOPK_RENORM, True, "last slot")
    # every layer routed its token to the bank's last slot
    assert all((ids[l] == E - 1).any() for l in range(L)), ids


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
    y_d = nm.DeviceBuffer(rows * H * 4)
    print(f"[stack ties rows={rows} mode={mode}]", flush=True)
    nm.stack_decode(layers, xd, rows, H, E, k, mode=mode, ids_out=ids_d, w_out=w_d, fused=True, y_out=y_d)
    nm.synchronize()
    assert nm.stack_status() == (0, 0)
    ids = ids_d.download(np.uint32).reshape(rows, k)
    w = w_d.download(np.float32).reshape(rows, k)
    want_ids, want_w, y = oracle_layer(host[0], x, E, k, mode, H)
    # the twins come out adjacent, even id first
    assert np.all(want_ids[:, 0::2] % 2 == 0) and np.array_equal(want_ids[:, 1::2], want_ids[:, 0::2] + 1)
    assert np.array_equal(ids, want_ids), (ids, want_ids)
    assert np.allclose(w, want_w, rtol=1e-5, atol=1e-7)
    assert S.max_rel_err(y_d.download(np.float32).reshape(rows, H), y) < TOL


@pytest.mark.parametrize("rows,E,k,dt", [
    (1, 128, 8, (O.Q4_K,) * 3),   # one token: the staged GEMV path
    (8, 128, 8, (O.Q4_K,) * 3),   # the matrix-core path
    (80, 128, 8, (O.Q4_K,) * 3),  # 640 pairs: the unstaged path (residual launch)
    (2, 64, 6, (O.Q4_K, O.Q4_K, O.Q8_0)),
])
def test_layered_residual_in_the_combine_is_bit_identical(gpu, rows, E, k, dt):
    """The layered chain without per-layer outputs adds each layer's residual in the
    decode's ordered combine; with them it keeps y and runs a residual launch.  Both
    give the same routing and the same final x, bit for bit."""
    nm = gpu
    H, L = 2048, 2
    I = 768 if dt[2] == O.Q4_K else 1408
    layers, host, keep = build_stack(nm, L, H, E, I, dt, 970 + rows)
    x = S.activations_bf16(971 + rows, rows, H)
    outs = []
    for want_y in (True, False):
        xd = nm.DeviceBuffer.from_array(x)
        ids_d = nm.DeviceBuffer(L * rows * k * 4)
        y_d = nm.DeviceBuffer(L * rows * H * 4) if want_y else None
        print(f"[layered residual rows={rows} E={E} k={k} y_out={want_y}]", flush=True)
        nm.stack_decode(layers, xd, rows, H, E, k, mode=O.ROUTE_SOFTMAX_TOPK_RENORM, ids_out=ids_d,
                        fused=False, y_out=y_d)
        nm.synchronize()
        outs.append((ids_d.download(np.uint32), xd.download(np.uint16)))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])


def test_fused_launches_on_two_streams_stay_ordered(gpu):
    """Two different two-layer Qwen3-shaped stacks launched alternately on two streams,
    eight launches with no host synchronisation between them: each launch uploads or
    reuses its own descriptor set on its stream and waits for the previous fused launch
    (they share the exchange words), so every launch's routing and outputs match the
    oracle layer by layer and no wait of the kernel runs out."""
    nm = gpu
    rows, L, H, E, k, I = 1, 2, 2048, 128, 8, 768
    dt = (O.Q4_K,) * 3
    stacks = [build_stack(nm, L, H, E, I, dt, 1400), build_stack(nm, L, H, E, I, dt, 1410)]
    streams = [nm.Stream(), nm.Stream()]
    mode = O.ROUTE_SOFTMAX_TOPK_RENORM
    runs = []
    for i in range(4):
        for j, (layers, host, keep) in enumerate(stacks):
            x = S.activations_bf16(1420 + 2 * i + j, rows, H)
            bufs = (nm.DeviceBuffer.from_array(x), nm.DeviceBuffer(L * rows * k * 4),
                    nm.DeviceBuffer(L * rows * k * 4), nm.DeviceBuffer(L * rows * H * 4))
            print(f"[two streams launch {i} stack {j}]", flush=True)
            nm.stack_decode(layers, bufs[0], rows, H, E, k, mode=mode, ids_out=bufs[1], w_out=bufs[2], fused=True,
                            y_out=bufs[3], stream=streams[j].handle)
            runs.append((j, x, bufs))
    for st in streams:
        st.sync()
    assert nm.stack_status() == (0, 0)
    for j, x, (xd, ids_d, w_d, y_d) in runs:
        host = stacks[j][1]
        check_chain(host, x, ids_d.download(np.uint32).reshape(L, rows, k), w_d.download(np.float32).reshape(L, rows, k),
                    y_d.download(np.float32).reshape(L, rows, H), xd.download(np.uint16).reshape(rows, H), rows, H,
                    E, k, mode)

