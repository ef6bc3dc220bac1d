"""The CPU baseline (oracle/cpu_baseline.c) that bench.py times beside the GPU.

It quantizes activations to int8 (per 256 values for Q4_K weights, per 32 for
Q8_0) like the reference's CPU path, so it is pinned here against an fp64
numpy restatement that applies the same activation rounding to x and to h:
a wrong scale, min, nibble half or block index moves the result far past the
bound.  Its distance from the exact oracle is the activation rounding alone."""
import numpy as np
import pytest

import cpu_baseline as CB
import oracle as O
import synthetic as S


def q8_round_trip(v: np.ndarray, block: int) -> np.ndarray:
    """Activation rounding of cpu_baseline.c in f32: per block d = amax / 127,
    q = rint(v * (127 / amax)) clamped to +-127, value = q * d."""
    v = np.asarray(v, dtype=np.float32).reshape(-1, block)
    amax = np.abs(v).max(axis=1, keepdims=True).astype(np.float32)
    safe = np.where(amax == 0, np.float32(1), amax)
    q = np.clip(np.rint(v * (np.float32(127) / safe)), -127, 127)
    d = (safe / np.float32(127)).astype(np.float32)
    return np.where(amax == 0, 0, q * d).reshape(-1)


def restated(g, u, d, dt, x, ids, w, H, I):
    gb = 256 if dt[0] == O.Q4_K else 32
    db = 256 if dt[2] == O.Q4_K else 32
    out = np.zeros((ids.shape[0], H), dtype=np.float64)
    for t in range(ids.shape[0]):
        xq = q8_round_trip(x[t], gb).astype(np.float64)
        for j in range(ids.shape[1]):
            if w[t, j] == 0:
                continue
            e = ids[t, j]
            G = O.dequantize_f64(dt[0], g[e], H).reshape(I, H)
            U = O.dequantize_f64(dt[1], u[e], H).reshape(I, H)
            D = O.dequantize_f64(dt[2], d[e], I).reshape(H, I)
            gv, uv = G @ xq, U @ xq
            h = gv / (1.0 + np.exp(-gv)) * uv
            out[t] += float(w[t, j]) * (D @ q8_round_trip(h, db).astype(np.float64))
    return out


@pytest.mark.parametrize("dt,E,H,I,k,rows", [
    ((O.Q4_K,) * 3, 8, 512, 256, 2, 2),
    ((O.Q8_0,) * 3, 8, 256, 512, 2, 3),
    ((O.Q4_K, O.Q4_K, O.Q8_0), 6, 512, 352, 3, 2),
])
def test_cpu_baseline_against_restatement(dt, E, H, I, k, rows):
    g, u, d, r = S.layer(31, E, H, I, dt)
    x = O.from_bf16(S.activations_bf16(32, rows, H))
    ids, w = O.topk(O.router_logits(x, r), k, O.ROUTE_SOFTMAX_TOPK_RENORM)
    w = w.copy()
    w[0, -1] = 0.0   # a zero weight is skipped
    st = (O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I))
    pool = CB.Pool(3)
    got = pool.fused_moe_decode(*st, x, ids, w)
    want = restated(g, u, d, dt, x, ids, w, H, I)
    # f32 accumulation over the same rounded activations (an h value near an
    # int8 rounding edge may round the other way in f32)
    assert S.max_rel_err(got, want) < 2e-3
    # the exact oracle differs by the activation rounding only
    exact = O.fused_moe_decode(*st, x, ids, w)
    assert S.max_rel_err(got, exact) < 5e-2


def test_cpu_baseline_pool_sizes_agree():
    dt = (O.Q4_K,) * 3
    E, H, I, k = 8, 512, 256, 2
    g, u, d, r = S.layer(33, E, H, I, dt)
    x = O.from_bf16(S.activations_bf16(34, 4, H))
    ids, w = O.topk(O.router_logits(x, r), k, O.ROUTE_SOFTMAX_TOPK_RENORM)
    st = (O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I))
    outs = [CB.Pool(n).fused_moe_decode(*st, x, ids, w) for n in (1, 2, 5)]
    # every unit computes the same sums in the same order whatever thread takes it
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_cpu_baseline_rejects_bad_ids():
    dt = (O.Q8_0,) * 3
    g, u, d, r = S.layer(35, 4, 64, 64, dt)
    st = (O.stack(g, dt[0], 64, 64), O.stack(u, dt[1], 64, 64), O.stack(d, dt[2], 64, 64))
    with pytest.raises(ValueError):
        CB.Pool(2).fused_moe_decode(*st, np.zeros((1, 64), np.float32), np.array([[4]], np.uint32),
                                    np.array([[1.0]], np.float32))
