"""Pins the CPU oracle (oracle/naiwa_oracle.c) before the GPU results are compared with it.

Every check here is independent of the oracle's own formulas: hand-built blocks
with hand-computed values, IEEE conversion known answers, round-trip bounds that
follow from the block format, an fp64 brute force cross-checked by numpy,
brute-force top-k and gather on tiny inputs, and the reference's own unit-test
fixtures and known answers (src/moe/tests.rs, src/prefill_stream.rs:1911-2002).
"""
import math

import numpy as np
import pytest

import oracle as O
import synthetic as S


# ---- scalar conversions (IEEE 754 binary16 / bfloat16, round to nearest even) ----

@pytest.mark.parametrize("value,bits", [
    (1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF), (65519.0, 0x7BFF), (65520.0, 0x7C00),
    (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0000), (3 * 2.0 ** -25, 0x0002),
    (1.0 + 2.0 ** -11, 0x3C00), (1.0 + 3 * 2.0 ** -11, 0x3C02), (0.1, 0x2E66),
    (float("inf"), 0x7C00), (6.103515625e-05, 0x0400),
])
def test_fp16_known_answers(value, bits):
    assert O.f32_to_fp16(value) == bits
    if bits != 0x7C00 or math.isinf(value):
        back = O.fp16_to_f32(bits)
        assert back == np.float32(np.float16(value)) or math.isinf(value)


def test_fp16_matches_numpy_on_a_sweep():
    x = O.normal(7, 20000, 0.0, 300.0)
    x = np.concatenate([x, O.normal(8, 2000, 0.0, 1e-5)])
    ours = np.array([O.f32_to_fp16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(ours, x.astype(np.float16).view(np.uint16))


def test_bf16_known_answers():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -0.0, 3.0e38], dtype=np.float32)
    assert O.to_bf16(x).tolist() == [0x3F80, 0x3F80, 0x3F82, 0x8000, 0x7F62]
    assert O.from_bf16(np.array([0x3F80, 0xC000], dtype=np.uint16)).tolist() == [1.0, -2.0]


# ---- block formats -----------------------------------------------------------------

def test_block_sizes_follow_ggml():
    # src/moe/tests.rs:101-107 ("Q8_0 (34 bytes a block of 32)") and src/moe/slot.rs:84-95
    assert O.row_bytes(O.Q8_0, 1024) == 32 * 34
    assert O.row_bytes(O.Q4_K, 2048) == 8 * 144
    assert O.row_bytes(O.Q4_K, 1408) == -1  # K % 256 != 0 is rejected (src/moe/expert.rs:130-135)
    assert O.row_bytes(O.Q8_0, 1408) == 44 * 34


def test_q8_0_hand_block():
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = [0x00, 0x34]  # d = 0.25
    blk[2:6] = np.array([-128, 127, 1, -1], dtype=np.int8).view(np.uint8)
    want = np.zeros(32, dtype=np.float32)
    want[:4] = [-32.0, 31.75, 0.25, -0.25]
    assert np.array_equal(O.dequantize(O.Q8_0, blk, 32), want)
    assert np.array_equal(O.dequantize_f64(O.Q8_0, blk, 32), want.astype(np.float64))


def q4k_hand_block():
    """d = 1, dmin = 0.5; sub-block 0: sc 3 m 2; 5: sc 37 m 21 (high bits in
    scales[1], scales[5]); 6: sc 63 m 63; every other scale and min is 0."""
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[2:4] = [0x00, 0x38]
    b[4:16] = [3, 0x80, 0xC0, 0, 2, 0x40, 0xC0, 0, 0, 0x55, 0xFF, 0]
    qs = b[16:]
    qs[0] = 0x0F          # element 0 (sub-block 0) nibble 15; element 32 nibble 0
    qs[64 + 3] = 0x70     # element 131 nibble 0 (sub-block 4), element 163 nibble 7 (sub-block 5)
    qs[96 + 5] = 0x03     # element 197 nibble 3 (sub-block 6)
    qs[96 + 31] = 0xA0    # element 255 nibble 10 (sub-block 7, scale 0)
    want = np.zeros(256, dtype=np.float32)
    want[0:32] = -1.0     # -dmin * 2
    want[0] = 44.0        # 1 * 3 * 15 - 1
    want[160:192] = -10.5  # -0.5 * 21
    want[163] = 248.5     # 37 * 7 - 10.5
    want[192:224] = -31.5  # -0.5 * 63
    want[197] = 157.5     # 63 * 3 - 31.5
    return b, want


def test_q4_k_hand_block():
    b, want = q4k_hand_block()
    assert np.array_equal(O.dequantize(O.Q4_K, b, 256), want)
    assert np.array_equal(O.dequantize_f64(O.Q4_K, b, 256), want.astype(np.float64))


def test_q4_k_all_zero_block():
    assert not O.dequantize(O.Q4_K, np.zeros(144, np.uint8), 256).any()


def test_q8_0_quantizer_round_trip_bound():
    x = O.normal(11, 64 * 32, 0.0, 0.02).reshape(64, 32)
    y = O.dequantize(O.Q8_0, O.quantize(O.Q8_0, x), 32)
    amax = np.abs(x).max(axis=1, keepdims=True)
    bound = amax * (1 / 254 + 1 / 2048) * (1 + 1e-6)
    assert (np.abs(y - x) <= bound).all()


def test_q4_k_quantizer_round_trip_bound():
    x = O.normal(12, 32 * 256, 0.0, 0.02).reshape(32, 256)
    y = O.dequantize(O.Q4_K, O.quantize(O.Q4_K, x), 256)
    err = np.abs(y - x)
    # within one 15-step quantum of the block's widest sub-block range
    sub = x.reshape(32, 8, 32)
    quantum = ((sub.max(axis=2) - np.minimum(sub.min(axis=2), 0)) / 15).max(axis=1)
    assert (err.max(axis=1) <= quantum).all()
    assert np.sqrt((err ** 2).mean()) < 0.2 * 0.02


def test_quantizers_are_deterministic():
    x = O.normal(13, 4 * 256)
    assert np.array_equal(O.quantize(O.Q4_K, x), O.quantize(O.Q4_K, x))


def test_normal_stream_is_counter_based():
    a = O.normal(5, 1000)
    b = O.normal(5, 500, offset=500)
    assert np.array_equal(a[500:], b)
    z = O.normal(6, 200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01


# ---- expert path ----------------------------------------------------------------------

def _stacks(g, u, d, H, I, dt):
    return (O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I))


def _numpy_reference(g, u, d, dt, H, I, xs, ids, w):
    """Independent fp64 restatement with numpy matmuls over dequantized experts."""
    E = g.shape[0]
    G = O.dequantize_f64(dt[0], g, H).reshape(E, I, H)
    U = O.dequantize_f64(dt[1], u, H).reshape(E, I, H)
    D = O.dequantize_f64(dt[2], d, I).reshape(E, H, I)
    out = np.zeros((xs.shape[0], H))
    for t in range(xs.shape[0]):
        x = xs[t].astype(np.float64)
        for j in range(ids.shape[1]):
            if w[t, j] == 0:
                continue
            e = ids[t, j]
            gx, ux = G[e] @ x, U[e] @ x
            h = gx / (1 + np.exp(-gx)) * ux
            out[t] += float(w[t, j]) * (D[e] @ h)
    return out


@pytest.mark.parametrize("dt,H,I", [((O.Q8_0,) * 3, 64, 32), ((O.Q4_K,) * 3, 256, 256),
                                    ((O.Q4_K, O.Q4_K, O.Q8_0), 256, 64)])
def test_fused_decode_against_fp64_and_numpy(dt, H, I):
    E, k, rows = 6, 3, 4
    g, u, d, _ = S.layer(21, E, H, I, dt, std=0.1)
    xs = O.normal(22, rows * H).reshape(rows, H)
    ids = np.array([[0, 3, 5], [2, 2, 1], [4, 0, 1], [5, 1, 3]], dtype=np.uint32)
    w = np.array([[0.5, 0.3, 0.2], [0.6, 0.0, 0.4], [0.1, 0.1, 0.8], [0.0, 0.0, 1.0]], np.float32)
    gs, us, ds = _stacks(g, u, d, H, I, dt)
    got = O.fused_moe_decode(gs, us, ds, xs, ids, w)
    f64 = O.fused_moe_decode_f64(gs, us, ds, xs, ids, w)
    ref = _numpy_reference(g, u, d, dt, H, I, xs, ids, w)
    assert S.max_rel_err(f64, ref) < 1e-10
    assert S.max_rel_err(got, f64) < 1e-5


def test_fused_decode_invariants():
    dt = (O.Q8_0,) * 3
    H, I, E = 64, 32, 8
    g, u, d, _ = S.layer(31, E, H, I, dt, std=0.1)
    gs, us, ds = _stacks(g, u, d, H, I, dt)
    xs = O.normal(32, H).reshape(1, H)
    ids = np.array([[1, 6]], np.uint32)
    w = np.array([[0.7, 0.3]], np.float32)
    base = O.fused_moe_decode(gs, us, ds, xs, ids, w)
    # weight-0 padding contributes exactly nothing (src/moe/stages/cpu_miss.rs:18-19)
    padded = O.fused_moe_decode(gs, us, ds, xs, np.array([[1, 6, 1]], np.uint32),
                                np.array([[0.7, 0.3, 0.0]], np.float32))
    assert np.array_equal(base, padded)
    # linear in the routing weights
    double = O.fused_moe_decode(gs, us, ds, xs, ids, w * 2)
    assert np.allclose(double, 2 * base, rtol=1e-6, atol=1e-7)
    # the slot order changes rounding only
    swapped = O.fused_moe_decode(gs, us, ds, xs, ids[:, ::-1].copy(), w[:, ::-1].copy())
    assert S.max_rel_err(swapped, base) < 1e-6
    # an out-of-range id is rejected, not read (src/moe/stages/route.rs:49-68)
    with pytest.raises(ValueError):
        O.fused_moe_decode(gs, us, ds, xs, np.array([[1, 8]], np.uint32), w)


def reference_fixture_stacks(e=8, hidden=64, inter=32):
    """The reference's test stacks: value i of a stacked [e, n, k] tensor is
    sin(i * 0.37 + seed) * 0.5, quantized to Q8_0 (src/moe/tests.rs:190-199,
    src/prefill_stream.rs:1801-1806)."""
    def q(n, k, seed):
        i = np.arange(e * n * k, dtype=np.float32)
        data = np.sin(i * np.float32(0.37) + np.float32(seed)).astype(np.float32) * np.float32(0.5)
        return O.quantize(O.Q8_0, data.reshape(e, n, k))
    return q(inter, hidden, 0.1), q(inter, hidden, 0.7), q(hidden, inter, 1.3)


def reference_fixture_xs(rows, hidden=64):
    return np.cos(np.arange(rows * hidden, dtype=np.float32) * np.float32(0.11)).reshape(rows, hidden)


@pytest.mark.parametrize("ids,ws,hits", [
    ([[0, 3]], [[0.6, 0.4]], {0, 2}),                              # src/moe/tests.rs:253-275
    ([[0, 3], [2, 0], [3, 5]], [[0.6, 0.4], [0.7, 0.3], [0.5, 0.5]], {0, 2}),  # :281-306
])
def test_reference_split_fixture(ids, ws, hits):
    """A resident/miss split of the routed experts sums to running every expert on
    the CPU (the reference's decode-split tests, tolerance 2e-2 there)."""
    g, u, d = reference_fixture_stacks()
    gs, us, ds = _stacks(g, u, d, 64, 32, (O.Q8_0,) * 3)
    ids = np.array(ids, np.uint32)
    ws = np.array(ws, np.float32)
    xs = reference_fixture_xs(ids.shape[0])
    full = O.fused_moe_decode(gs, us, ds, xs, ids, ws)
    hit_w = np.where(np.isin(ids, list(hits)), ws, 0).astype(np.float32)
    miss_w = (ws - hit_w).astype(np.float32)
    split = O.fused_moe_decode(gs, us, ds, xs, ids, hit_w) + O.fused_moe_decode(gs, us, ds, xs, ids, miss_w)
    assert np.abs(split - full).max() < 1e-5
    # a swapped weight moves the output by far more than the tolerance (the test's own control)
    bad = O.fused_moe_decode(gs, us, ds, xs, ids, ws[:, ::-1].copy())
    assert np.abs(bad - full).max() > 2e-2


def test_reference_prefill_fixture():
    """src/prefill_stream.rs:1911-2002: E=4, hidden 64, inter 32, 3 tokens, full
    top-k and a one-expert subset, against per-expert dequantized products."""
    g, u, d = reference_fixture_stacks(e=4)
    dt = (O.Q8_0,) * 3
    gs, us, ds = _stacks(g, u, d, 64, 32, dt)
    xs = reference_fixture_xs(3)
    ids = np.array([[0, 2], [3, 1], [2, 0]], np.uint32)
    ws = np.array([[0.6, 0.4], [0.3, 0.7], [0.5, 0.5]], np.float32)
    for sub in (2, 1):
        i, w = ids[:, :sub].copy(), ws[:, :sub].copy()
        got = O.fused_moe_decode(gs, us, ds, xs, i, w)
        want = _numpy_reference(g, u, d, dt, 64, 32, xs, i, w)
        assert np.abs(got - want).max() < 1e-4


# ---- router ---------------------------------------------------------------------------

def test_topk_known_answers():
    # src/moe/tests.rs:169-173
    ids, _ = O.topk(np.array([[0.1, 0.9, 0.5, 0.9]], np.float32), 3)
    assert ids.tolist() == [[1, 3, 2]]
    ids, _ = O.topk(np.array([[1.0, 2.0]], np.float32), 2)
    assert ids.tolist() == [[1, 0]]


def test_topk_brute_force_with_ties():
    rng = np.random.default_rng(3)
    for trial in range(50):
        E = int(rng.integers(2, 40))
        k = int(rng.integers(1, E + 1))
        l = rng.integers(-3, 4, size=(3, E)).astype(np.float32)  # many ties
        ids, w = O.topk(l, k, O.ROUTE_SOFTMAX_TOPK_RENORM)
        for t in range(3):
            want = sorted(range(E), key=lambda e: (-l[t, e], e))[:k]
            assert ids[t].tolist() == want
            ex = np.exp(l[t, want].astype(np.float64) - l[t, want[0]])
            assert np.allclose(w[t], ex / ex.sum(), rtol=1e-6)


def test_topk_modes():
    l = np.array([[2.0, 1.0, 0.5, -1.0]], np.float32)
    _, w_renorm = O.topk(l, 2, O.ROUTE_SOFTMAX_TOPK_RENORM)
    _, w_mixtral = O.topk(l, 2, O.ROUTE_TOPK_SOFTMAX)
    _, w_all = O.topk(l, 2, O.ROUTE_SOFTMAX_TOPK)
    e = np.exp(l[0].astype(np.float64) - 2.0)
    assert np.allclose(w_renorm[0], e[:2] / e[:2].sum(), rtol=1e-6)
    assert np.array_equal(w_renorm, w_mixtral)
    assert np.allclose(w_all[0], e[:2] / e.sum(), rtol=1e-6)


def test_router_logits_against_fp64():
    x = O.from_bf16(S.activations_bf16(41, 3, 2048))
    W = O.normal(42, 128 * 2048, 0.0, 0.02).reshape(128, 2048)
    got = O.router_logits(x, W)
    exact = x.astype(np.float64) @ W.astype(np.float64).T
    bound = 1e-6 * (np.abs(x).astype(np.float64) @ np.abs(W).astype(np.float64).T) + 256 * 2.0 ** -32
    assert (np.abs(got - exact) <= bound + np.abs(exact) * 2 ** -23).all()


def test_router_logits_chunk_order_independent():
    """Reversing the feature order inside every chunk changes the f32 partials; reversing
    the chunk order must not change anything (partials are added as integers)."""
    x = O.from_bf16(S.activations_bf16(43, 2, 512))
    W = O.normal(44, 16 * 512, 0.0, 0.02).reshape(16, 512)
    base = O.router_logits(x, W)
    perm = np.arange(512).reshape(64, 8)[::-1].reshape(-1)
    assert np.array_equal(O.router_logits(x[:, perm].copy(), W[:, perm].copy()), base)


def test_stack_decode_is_residual_chain():
    H, I, E, k = 256, 256, 4, 2
    layers = []
    for l in range(2):
        g, u, d, r = S.layer(50 + l, E, H, I)
        layers.append((r, (g, u, d), (O.Q4_K,) * 3, I))
    x0 = S.activations_bf16(52, 2, H)
    x1, ids, w = O.stack_decode(layers, x0, E, k)
    # replay layer by layer with the single-layer functions
    x = O.from_bf16(x0)
    for l, (r, (g, u, d), dt, _) in enumerate(layers):
        lg = O.router_logits(x, r)
        i, ww = O.topk(lg, k)
        assert np.array_equal(i, ids[l]) and np.array_equal(ww, w[l])
        gs, us, ds = _stacks(g, u, d, H, I, dt)
        y = O.fused_moe_decode(gs, us, ds, x, i, ww)
        x = O.from_bf16(O.to_bf16(x + y))
    assert np.array_equal(O.to_bf16(x), x1)


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_threaded_expert_path_is_bit_identical(threads):
    """The CPU baseline's threaded expert path splits rows and features over
    threads but computes every value as the single-threaded pass does."""
    H, I, E, k = 512, 256, 8, 3
    g, u, d, r = S.layer(60, E, H, I, (O.Q4_K, O.Q4_K, O.Q8_0))
    gs, us, ds = _stacks(g, u, d, H, I, (O.Q4_K, O.Q4_K, O.Q8_0))
    x = O.from_bf16(S.activations_bf16(61, 3, H))
    ids = np.array([[1, 5, 1], [7, 0, 2], [3, 3, 6]], dtype=np.uint32)   # repeats share pass 1
    w = np.array([[0.5, 0.25, 0.25], [0.0, 0.6, 0.4], [0.3, 0.3, 0.4]], dtype=np.float32)
    want = O.fused_moe_decode(gs, us, ds, x, ids, w)
    assert np.array_equal(O.fused_moe_decode_mt(gs, us, ds, x, ids, w, threads), want)
    layers = [(r, (g, u, d), (O.Q4_K, O.Q4_K, O.Q8_0), I)]
    x0 = S.activations_bf16(62, 2, H)
    a = O.stack_decode(layers, x0, E, 2)
    b = O.stack_decode(layers, x0, E, 2, threads=threads)
    assert all(np.array_equal(p, q) for p, q in zip(a, b))


# ---- gather ---------------------------------------------------------------------------

def test_gather_brute_force():
    rng = np.random.default_rng(9)
    for _ in range(30):
        E = int(rng.integers(1, 70))
        n = int(rng.integers(0, 300))
        ids = rng.integers(0, E, size=n).astype(np.uint32)
        perm, off = O.gather(ids, E)
        want = sorted(range(n), key=lambda i: (ids[i], i))
        assert perm.tolist() == want
        counts = np.bincount(ids, minlength=E)
        assert off.tolist() == [0] + np.cumsum(counts).tolist()


def test_gather_rejects_bad_ids():
    with pytest.raises(ValueError):
        O.gather(np.array([0, 5], np.uint32), 5)
