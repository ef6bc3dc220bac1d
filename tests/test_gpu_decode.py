"""GPU parity of naiwa_moe_decode (the indexed_moe_fused_decode replacement) against
the CPU oracle on the same seeded bytes.  Bar: max relative error 1e-2 (norm-relative,
f32 accumulation), the tolerance of the north-star parity contract."""
import numpy as np
import pytest

import oracle as O
import synthetic as S

TOL = 1e-2

pytestmark = pytest.mark.gpu


def run_decode(nm, g, u, d, dt, H, I, x_bf16, slot_ids, w, slots_of_expert=None, act=0,
               x_f32=False):
    """Upload the experts into slot banks (expert e -> slot slots_of_expert[e]) and run."""
    E = g.shape[0]
    if slots_of_expert is None:
        slots_of_expert = list(range(E))
    nslots = max(slots_of_expert) + 1
    banks = nm.LayerBanks(nslots, H, I, dt)
    for e, s in enumerate(slots_of_expert):
        banks.load(s, g[e], u[e], d[e])
    rows, width = slot_ids.shape
    if x_f32:
        xd = nm.DeviceBuffer.from_array(O.from_bf16(x_bf16))
        xdt = nm.F32
    else:
        xd = nm.DeviceBuffer.from_array(x_bf16)
        xdt = nm.BF16
    ids_d = nm.DeviceBuffer.from_array(np.ascontiguousarray(slot_ids, np.uint32))
    w_d = nm.DeviceBuffer.from_array(np.ascontiguousarray(w, np.float32))
    out = nm.DeviceBuffer(rows * H * 4)
    nm.indexed_moe_fused_decode(banks, xd, xdt, ids_d, w_d, rows, width, out, act=act)
    nm.synchronize()
    return out.download(np.float32).reshape(rows, H)


def oracle_decode(g, u, d, dt, H, I, x_bf16, ids, w):
    gs, us, ds = (O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I))
    return O.fused_moe_decode(gs, us, ds, O.from_bf16(x_bf16), ids, w)


def test_c1_mixtral_style_q8_0_layer(gpu):
    """hidden 1024, 8 experts, top-2, intermediate 2048, Q8_0, 1 token, seed 0."""
    nm = gpu
    H, I, E, k = 1024, 2048, 8, 2
    dt = (O.Q8_0,) * 3
    g, u, d, r = S.layer(0, E, H, I, dt)
    x = S.activations_bf16(0, 1, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k, O.ROUTE_TOPK_SOFTMAX)
    print(f"[c1] ids={ids.tolist()} w={w.tolist()}", flush=True)
    got = run_decode(nm, g, u, d, dt, H, I, x, ids, w)
    want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    err = S.max_rel_err(got, want)
    print(f"[c1] max_rel_err={err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("rows", [1, 3, 8])
def test_qwen3_shape_q4_k(gpu, rows):
    """Qwen3-30B-A3B expert shape (hidden 2048, intermediate 768, Q4_K, top-8) on 24 experts."""
    nm = gpu
    H, I, E, k = 2048, 768, 24, 8
    dt = (O.Q4_K,) * 3
    g, u, d, r = S.layer(100 + rows, E, H, I, dt)
    x = S.activations_bf16(100 + rows, rows, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k)
    got = run_decode(nm, g, u, d, dt, H, I, x, ids, w)
    want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    err = S.max_rel_err(got, want)
    print(f"[qwen3 rows={rows}] max_rel_err={err:.3e}", flush=True)
    assert err < TOL


def test_mixed_formats_deepseek_shape(gpu):
    """gate/up Q4_K, down Q8_0 at intermediate 1408 (K=1408 is not a Q4_K multiple)."""
    nm = gpu
    H, I, E, k = 2048, 1408, 10, 6
    dt = (O.Q4_K, O.Q4_K, O.Q8_0)
    g, u, d, r = S.layer(200, E, H, I, dt)
    x = S.activations_bf16(200, 4, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k, O.ROUTE_SOFTMAX_TOPK)
    got = run_decode(nm, g, u, d, dt, H, I, x, ids, w)
    want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    assert S.max_rel_err(got, want) < TOL


def test_slot_indexing_padding_and_shared_experts(gpu):
    """Experts sit in permuted slots; rows share experts; weight-0 pads (the
    reference's padding, src/moe/stages/gpu.rs:117-129) contribute nothing."""
    nm = gpu
    H, I, E = 256, 256, 6
    dt = (O.Q4_K,) * 3
    g, u, d, _ = S.layer(300, E, H, I, dt, std=0.1)
    x = S.activations_bf16(300, 4, H)
    ids = np.array([[0, 3, 5], [3, 3, 1], [4, 0, 0], [2, 5, 3]], np.uint32)
    w = np.array([[0.5, 0.3, 0.2], [0.6, 0.0, 0.4], [0.9, 0.1, 0.0], [0.2, 0.2, 0.6]], np.float32)
    slot_of = [4, 0, 7, 2, 1, 5]
    slot_ids = np.vectorize(lambda e: slot_of[e])(ids).astype(np.uint32)
    got = run_decode(nm, g, u, d, dt, H, I, x, slot_ids, w, slots_of_expert=slot_of)
    want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    assert S.max_rel_err(got, want) < TOL


def test_f32_activations_and_gelu(gpu):
    nm = gpu
    H, I, E = 512, 256, 4
    dt = (O.Q8_0,) * 3
    g, u, d, _ = S.layer(400, E, H, I, dt, std=0.05)
    x = S.activations_bf16(400, 2, H)
    ids = np.array([[1, 2], [3, 0]], np.uint32)
    w = np.array([[0.7, 0.3], [0.4, 0.6]], np.float32)
    got = run_decode(nm, g, u, d, dt, H, I, x, ids, w, x_f32=True)
    want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    assert S.max_rel_err(got, want) < TOL
    # GELU(tanh) path against an fp64 numpy restatement
    got_g = run_decode(nm, g, u, d, dt, H, I, x, ids, w, act=1)
    G = O.dequantize_f64(dt[0], g, H).reshape(E, I, H)
    U = O.dequantize_f64(dt[1], u, H).reshape(E, I, H)
    D = O.dequantize_f64(dt[2], d, I).reshape(E, H, I)
    xf = O.from_bf16(x).astype(np.float64)
    want_g = np.zeros((2, H))
    for t in range(2):
        for j in range(2):
            e = ids[t, j]
            gx = G[e] @ xf[t]
            gel = 0.5 * gx * (1 + np.tanh(np.sqrt(2 / np.pi) * (gx + 0.044715 * gx ** 3)))
            want_g[t] += w[t, j] * (D[e] @ (gel * (U[e] @ xf[t])))
    assert S.max_rel_err(got_g, want_g) < TOL


def test_empty_and_all_padding(gpu):
    nm = gpu
    H, I, E = 256, 256, 2
    dt = (O.Q4_K,) * 3
    g, u, d, _ = S.layer(500, E, H, I, dt)
    x = S.activations_bf16(500, 2, H)
    ids = np.array([[1, 1], [0, 0]], np.uint32)
    w = np.zeros((2, 2), np.float32)
    got = run_decode(nm, g, u, d, dt, H, I, x, ids, w)
    assert not got.any()


def test_reference_split_fixture_on_gpu(gpu):
    """src/moe/tests.rs:253-306 on the device: the resident experts run on the GPU
    banks, the misses on the CPU oracle; the sum matches all-CPU within 2e-2
    (the reference's bound), and within the 1e-2 relative bar of these tests."""
    import test_oracle as T
    nm = gpu
    g, u, d = T.reference_fixture_stacks()
    dt = (O.Q8_0,) * 3
    for ids, ws in (([[0, 3]], [[0.6, 0.4]]),
                    ([[0, 3], [2, 0], [3, 5]], [[0.6, 0.4], [0.7, 0.3], [0.5, 0.5]])):
        ids = np.array(ids, np.uint32)
        ws = np.array(ws, np.float32)
        xs = T.reference_fixture_xs(ids.shape[0])
        x_bf16 = O.to_bf16(xs)
        resident = {0: 0, 2: 1}  # experts 0 and 2 admitted (slots 0, 1)
        hit = np.isin(ids, list(resident))
        slot_ids = np.where(hit, np.vectorize(lambda e: resident.get(int(e), 0))(ids), 0).astype(np.uint32)
        hit_w = np.where(hit, ws, 0).astype(np.float32)
        banks_g = np.stack([g[0], g[2]]); banks_u = np.stack([u[0], u[2]]); banks_d = np.stack([d[0], d[2]])
        gpu_part = run_decode(nm, banks_g, banks_u, banks_d, dt, 64, 32, x_bf16, slot_ids, hit_w)
        cpu_part = oracle_decode(g, u, d, dt, 64, 32, x_bf16, ids, (ws - hit_w).astype(np.float32))
        full = oracle_decode(g, u, d, dt, 64, 32, x_bf16, ids, ws)
        assert np.abs(gpu_part + cpu_part - full).max() < 2e-2
        assert S.max_rel_err(gpu_part + cpu_part, full) < TOL


def test_decode_is_deterministic(gpu):
    nm = gpu
    H, I, E, k = 2048, 768, 16, 8
    dt = (O.Q4_K,) * 3
    g, u, d, r = S.layer(600, E, H, I, dt)
    x = S.activations_bf16(600, 4, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k)
    a = run_decode(nm, g, u, d, dt, H, I, x, ids, w)
    b = run_decode(nm, g, u, d, dt, H, I, x, ids, w)
    assert np.array_equal(a, b)


def test_split_by_slot_with_accumulate_is_bit_identical(gpu):
    """A call over the pairs of low slots, then an accumulating call over the pairs of
    higher slots, equals one call over all pairs bit for bit (the partial-cache step runs
    the cache slots while the staged ones are still landing)."""
    nm = gpu
    H, I, E, k, rows = 512, 256, 12, 4, 5
    dt = (O.Q4_K, O.Q4_K, O.Q8_0)
    g, u, d, r = S.layer(2100, E, H, I, dt)
    banks = nm.LayerBanks(E, H, I, dt)
    for e in range(E):
        banks.load(e, g[e], u[e], d[e])
    x = S.activations_bf16(2101, rows, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k)
    xd, idd = nm.DeviceBuffer.from_array(x), nm.DeviceBuffer.from_array(ids.astype(np.uint32))
    whole, split = nm.DeviceBuffer(rows * H * 4), nm.DeviceBuffer(rows * H * 4)
    nm.indexed_moe_fused_decode(banks, xd, nm.BF16, idd, nm.DeviceBuffer.from_array(w), rows, k, whole)
    for cut in (3, 7, 11):
        lo = nm.DeviceBuffer.from_array(np.where(ids < cut, w, 0.0).astype(np.float32))
        hi = nm.DeviceBuffer.from_array(np.where(ids >= cut, w, 0.0).astype(np.float32))
        nm.indexed_moe_fused_decode(banks, xd, nm.BF16, idd, lo, rows, k, split)
        nm.indexed_moe_fused_decode(banks, xd, nm.BF16, idd, hi, rows, k, split, accumulate=True)
        nm.synchronize()
        assert np.array_equal(whole.download(np.float32), split.download(np.float32)), cut


@pytest.mark.parametrize("dt,H,I,E,k", [
    ((O.Q4_K,) * 3, 2048, 768, 16, 8),              # one K part, 8 pairs
    ((O.Q4_K,) * 3, 1024, 4352, 8, 2),              # three K parts: 2048 + 2048 + 256
    ((O.Q4_K, O.Q4_K, O.Q8_0), 512, 2304, 6, 4),    # Q8_0 down in two K parts
    ((O.Q4_K, O.Q4_K, O.Q8_0), 1024, 1408, 12, 6),  # Q8_0 down in one K part (one launch for down + combine)
    ((O.Q8_0,) * 3, 512, 1376, 20, 16),             # odd Q8_0 block count, 16 pairs (one launch)
])
def test_one_token_combine_matches_the_general_combine(gpu, dt, H, I, E, k):
    """A one-token call (its combine issues every load up front, or down and combine run
    as one launch when the down rows fit one K part) gives row 0 of a two-token call
    over the same pairs (the general combine) bit for bit, plain and accumulating into
    an output that already holds values."""
    nm = gpu
    g, u, d, r = S.layer(2200 + H, E, H, I, dt)
    banks = nm.LayerBanks(E, H, I, dt)
    for e in range(E):
        banks.load(e, g[e], u[e], d[e])
    x = S.activations_bf16(2201, 2, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k)
    base = np.random.default_rng(2202).standard_normal((2, H)).astype(np.float32)
    res = {}
    for rows in (1, 2):
        xd = nm.DeviceBuffer.from_array(np.ascontiguousarray(x[:rows]))
        idd = nm.DeviceBuffer.from_array(np.ascontiguousarray(ids[:rows], np.uint32))
        wd = nm.DeviceBuffer.from_array(np.ascontiguousarray(w[:rows], np.float32))
        plain = nm.DeviceBuffer(rows * H * 4)
        acc = nm.DeviceBuffer.from_array(np.ascontiguousarray(base[:rows]))
        nm.indexed_moe_fused_decode(banks, xd, nm.BF16, idd, wd, rows, k, plain)
        nm.indexed_moe_fused_decode(banks, xd, nm.BF16, idd, wd, rows, k, acc, accumulate=True)
        nm.synchronize()
        res[rows] = (plain.download(np.float32).reshape(rows, H), acc.download(np.float32).reshape(rows, H))
    assert np.array_equal(res[1][0][0], res[2][0][0])
    assert np.array_equal(res[1][1][0], res[2][1][0])
    want = oracle_decode(g, u, d, dt, H, I, x[:1], ids[:1], w[:1])
    assert S.max_rel_err(res[1][0], want) < TOL


@pytest.mark.parametrize("dt,H,I,E,k,rows", [
    ((O.Q4_K,) * 3, 512, 2304, 4, 2, 3),             # down in two K parts: 2048 + 256
    ((O.Q8_0,) * 3, 256, 2080, 4, 2, 5),             # 65 Q8_0 blocks a row: parts of 2048 + 32
    ((O.Q4_K, O.Q4_K, O.Q8_0), 256, 6144, 3, 2, 9),  # three full parts, 9 tokens (two passes of 8)
    ((O.Q4_K,) * 3, 256, 512, 24, 20, 2),            # 20 pairs a token: the f32-h path
    ((O.Q4_K,) * 3, 256, 256, 16, 8, 80),            # 640 pairs: the f32-h path
])
def test_k_parts_and_large_calls(gpu, dt, H, I, E, k, rows):
    """The down projection split into K parts of 2048 (a short last part, odd Q8_0
    block counts, token passes), and the calls past the staged path's limits."""
    nm = gpu
    g, u, d, r = S.layer(2300 + I + rows, E, H, I, dt)
    x = S.activations_bf16(2300 + rows, rows, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k)
    print(f"[k parts H={H} I={I} E={E} k={k} rows={rows}]", flush=True)
    got = run_decode(nm, g, u, d, dt, H, I, x, ids, w)
    want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    err = S.max_rel_err(got, want)
    print(f"  max_rel_err={err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("dt,H,I,E,k,rows,x_f32,act", [
    ((O.Q8_0,) * 3, 512, 256, 4, 2, 40, False, 0),            # ~20 tokens a slot: two 16-token chunks
    ((O.Q4_K,) * 3, 256, 512, 3, 2, 33, True, 0),             # f32 activations, three chunks
    ((O.Q4_K, O.Q4_K, O.Q8_0), 512, 384, 6, 3, 12, False, 1),  # GELU(tanh), mixed formats
    ((O.Q8_0, O.Q8_0, O.Q4_K), 384, 2304, 5, 2, 7, False, 0),  # Q4_K down in two K parts
])
def test_matrix_core_decode(gpu, dt, H, I, E, k, rows, x_f32, act):
    """Calls of 4 or more rows run their expert GEMMs on the matrix cores (bf16
    operands, f32 accumulation): every format pairing, tokens past one 16-token
    tile, K parts of the down projection, f32 input and both activations."""
    nm = gpu
    g, u, d, r = S.layer(2500 + rows, E, H, I, dt)
    x = S.activations_bf16(2500 + rows, rows, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k)
    print(f"[mfma decode dt={dt} H={H} I={I} rows={rows} act={act}]", flush=True)
    got = run_decode(nm, g, u, d, dt, H, I, x, ids, w, act=act, x_f32=x_f32)
    if act == 0:
        want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    else:
        G = O.dequantize_f64(dt[0], g, H).reshape(E, I, H)
        U = O.dequantize_f64(dt[1], u, H).reshape(E, I, H)
        D = O.dequantize_f64(dt[2], d, I).reshape(E, H, I)
        xf = O.from_bf16(x).astype(np.float64)
        want = np.zeros((rows, H))
        for t in range(rows):
            for j in range(k):
                e = ids[t, j]
                gx = G[e] @ xf[t]
                gel = 0.5 * gx * (1 + np.tanh(np.sqrt(2 / np.pi) * (gx + 0.044715 * gx ** 3)))
                want[t] += w[t, j] * (D[e] @ (gel * (U[e] @ xf[t])))
    err = S.max_rel_err(got, want)
    print(f"  max_rel_err={err:.3e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("x_f32", [False, True])
def test_matrix_core_decode_takes_activations_of_1e5(gpu, x_f32):
    """The matrix-core decode (8 rows) with every other token's activations scaled
    to ~1e5 (h then reaches ~1e9, far past the f16 range): bf16 operands keep the
    exponent range, so both groups of rows land within the 1e-2 bar of the oracle,
    each against its own scale."""
    nm = gpu
    dt, H, I, E, k, rows = (O.Q4_K, O.Q4_K, O.Q8_0), 512, 384, 6, 3, 8
    g, u, d, r = S.layer(2600, E, H, I, dt)
    x0 = S.activations_bf16(2601, rows, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x0), r), k)
    xs = O.from_bf16(x0).copy()
    big = np.arange(rows) % 2 == 0
    xs[big] *= np.float32(1.0e5)
    x = O.to_bf16(xs)
    print(f"[mfma decode 1e5 rows x_f32={x_f32}]", flush=True)
    got = run_decode(nm, g, u, d, dt, H, I, x, ids, w, x_f32=x_f32)
    want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    assert np.isfinite(got).all()
    assert np.abs(want[big]).max() > 1.0e8
    for sel in (big, ~big):
        err = S.max_rel_err(got[sel], want[sel])
        print(f"  max_rel_err={err:.3e}", flush=True)
        assert err < TOL


def test_matrix_core_decode_accumulates(gpu):
    """NAIWA_DECODE_ACCUMULATE on the matrix-core path adds to out's values."""
    nm = gpu
    dt = (O.Q4_K,) * 3
    H, I, E, k, rows = 256, 256, 4, 2, 9
    g, u, d, r = S.layer(2600, E, H, I, dt)
    banks = nm.LayerBanks(E, H, I, dt)
    for e in range(E):
        banks.load(e, g[e], u[e], d[e])
    x = S.activations_bf16(2601, rows, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k)
    start = np.linspace(-1, 1, rows * H, dtype=np.float32).reshape(rows, H)
    out = nm.DeviceBuffer.from_array(start)
    nm.indexed_moe_fused_decode(banks, nm.DeviceBuffer.from_array(x), nm.BF16,
                                nm.DeviceBuffer.from_array(ids.astype(np.uint32)),
                                nm.DeviceBuffer.from_array(w), rows, k, out, accumulate=True)
    nm.synchronize()
    got = out.download(np.float32).reshape(rows, H) - start
    assert S.max_rel_err(got, oracle_decode(g, u, d, dt, H, I, x, ids, w)) < TOL


@pytest.mark.parametrize("rows", [1, 2, 3])
def test_small_calls_segment_in_the_expert_kernel(gpu, rows):
    """Calls of at most 64 pairs below 4 rows are grouped by slot inside the gate/up
    launch: repeated slots in a row and across rows, weight-0 padding and permuted
    slots give the oracle's sums."""
    nm = gpu
    H, I, E, width = 256, 512, 6, 5
    dt = (O.Q4_K,) * 3
    g, u, d, _ = S.layer(2700 + rows, E, H, I, dt, std=0.1)
    x = S.activations_bf16(2700 + rows, rows, H)
    ids = np.array([[2, 2, 5, 0, 3], [5, 1, 1, 4, 2], [0, 3, 3, 3, 5]], np.uint32)[:rows]
    w = np.array([[0.3, 0.2, 0.1, 0.0, 0.4], [0.5, 0.25, 0.0, 0.15, 0.1], [0.2, 0.2, 0.2, 0.2, 0.2]],
                 np.float32)[:rows]
    slot_of = [3, 0, 5, 1, 4, 2]
    slot_ids = np.vectorize(lambda e: slot_of[e])(ids).astype(np.uint32)
    got = run_decode(nm, g, u, d, dt, H, I, x, slot_ids, w, slots_of_expert=slot_of)
    want = oracle_decode(g, u, d, dt, H, I, x, ids, w)
    assert S.max_rel_err(got, want) < TOL
