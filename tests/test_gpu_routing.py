"""GPU router top-k and gather: bit-exact against the oracle (ids, logits,
permutations, offsets), ties broken by the lower expert id."""
import numpy as np
import pytest

import oracle as O
import synthetic as S

pytestmark = pytest.mark.gpu


def gpu_router(nm, x_bf16, W, k, mode, x_f32=False):
    rows, H = x_bf16.shape
    E = W.shape[0]
    if x_f32:
        xd, xdt = nm.DeviceBuffer.from_array(O.from_bf16(x_bf16)), nm.F32
    else:
        xd, xdt = nm.DeviceBuffer.from_array(x_bf16), nm.BF16
    Wd = nm.DeviceBuffer.from_array(np.ascontiguousarray(W, np.float32))
    ids = nm.DeviceBuffer(rows * k * 4)
    w = nm.DeviceBuffer(rows * k * 4)
    logits = nm.DeviceBuffer(rows * E * 4)
    nm.router_topk(xd, xdt, Wd, rows, H, E, k, ids, w, mode=mode, logits_out=logits)
    nm.synchronize()
    return (ids.download(np.uint32).reshape(rows, k), w.download(np.float32).reshape(rows, k),
            logits.download(np.float32).reshape(rows, E))


@pytest.mark.parametrize("rows,H,E,k,mode", [
    (1, 2048, 128, 8, O.ROUTE_SOFTMAX_TOPK_RENORM),   # Qwen3-30B-A3B
    (8, 2048, 128, 8, O.ROUTE_SOFTMAX_TOPK_RENORM),
    (1, 1024, 8, 2, O.ROUTE_TOPK_SOFTMAX),            # Mixtral-style C1
    (16, 4096, 8, 2, O.ROUTE_TOPK_SOFTMAX),           # Mixtral-8x7B
    (5, 2048, 64, 6, O.ROUTE_SOFTMAX_TOPK),           # DeepSeek-V2-Lite
    (3, 512, 1000, 32, O.ROUTE_SOFTMAX_TOPK_RENORM),  # wide E, large k
    (512, 2048, 64, 6, O.ROUTE_SOFTMAX_TOPK),         # a DeepSeek-V2-Lite prefill chunk (tiled kernel)
    (100, 4096, 8, 2, O.ROUTE_TOPK_SOFTMAX),          # Mixtral prefill rows, ragged row tile
    (70, 2048, 130, 8, O.ROUTE_SOFTMAX_TOPK_RENORM),  # 16-row blocks, 5 row groups
    (300, 4096, 16, 2, O.ROUTE_TOPK_SOFTMAX),         # 16-row blocks at H 4096
    (40, 1024, 128, 8, O.ROUTE_SOFTMAX_TOPK_RENORM),  # 16-row blocks at another H
])
def test_router_bit_exact(gpu, rows, H, E, k, mode):
    x = S.activations_bf16(700 + rows, rows, H)
    W = O.normal(701 + E, E * H, 0.0, 0.02).reshape(E, H)
    ids, w, logits = gpu_router(gpu, x, W, k, mode)
    want_logits = O.router_logits(O.from_bf16(x), W)
    want_ids, want_w = O.topk(want_logits, k, mode)
    assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
    assert np.array_equal(ids, want_ids)
    assert np.allclose(w, want_w, rtol=1e-5, atol=1e-7)


def test_router_ties_go_to_the_lower_id(gpu):
    """Identical router rows give identical logits: the lower expert id ranks first."""
    H, E, k = 256, 16, 6
    W = O.normal(720, E * H, 0.0, 0.02).reshape(E, H)
    W[9] = W[2]
    W[14] = W[2]
    W[5] = W[11]
    x = S.activations_bf16(721, 4, H)
    ids, _, logits = gpu_router(gpu, x, W, k, O.ROUTE_SOFTMAX_TOPK_RENORM)
    want_ids, _ = O.topk(O.router_logits(O.from_bf16(x), W), k)
    assert np.array_equal(ids, want_ids)
    for t in range(4):
        assert logits[t, 2] == logits[t, 9] == logits[t, 14]
        row = ids[t].tolist()
        if 9 in row:
            assert 2 in row and row.index(2) < row.index(9)


def test_router_f32_input(gpu):
    x = S.activations_bf16(730, 2, 1024)
    W = O.normal(731, 8 * 1024, 0.0, 0.02).reshape(8, 1024)
    ids, _, logits = gpu_router(gpu, x, W, 2, O.ROUTE_TOPK_SOFTMAX, x_f32=True)
    want = O.router_logits(O.from_bf16(x), W)
    assert np.array_equal(logits, want)
    assert np.array_equal(ids, O.topk(want, 2, O.ROUTE_TOPK_SOFTMAX)[0])


@pytest.mark.parametrize("n,E", [(0, 8), (1, 128), (8, 128), (64, 128), (2048, 128), (300, 4096),
                                 (5000, 7)])
def test_gather_bit_exact(gpu, n, E):
    nm = gpu
    rng = np.random.default_rng(n * 31 + E)
    ids = rng.integers(0, E, size=n).astype(np.uint32)
    idsd = nm.DeviceBuffer.from_array(ids) if n else nm.DeviceBuffer(4)
    perm = nm.DeviceBuffer(max(n, 1) * 4)
    off = nm.DeviceBuffer((E + 1) * 4)
    bad = nm.DeviceBuffer(4)
    nm.moe_gather(idsd, n, E, perm, off, bad)
    nm.synchronize()
    want_perm, want_off = O.gather(ids, E)
    assert np.array_equal(perm.download(np.uint32, n), want_perm)
    assert np.array_equal(off.download(np.uint32), want_off)
    assert bad.download(np.int32)[0] == 0


def test_gather_counts_out_of_range_ids(gpu):
    nm = gpu
    ids = np.array([3, 9, 1, 3, 12, 0], np.uint32)
    perm = nm.DeviceBuffer(6 * 4)
    off = nm.DeviceBuffer(9 * 4)
    bad = nm.DeviceBuffer(4)
    nm.moe_gather(nm.DeviceBuffer.from_array(ids), 6, 8, perm, off, bad)
    nm.synchronize()
    assert bad.download(np.int32)[0] == 2
    assert perm.download(np.uint32, 4).tolist() == [5, 2, 0, 3]
    assert off.download(np.uint32).tolist() == [0, 1, 2, 2, 4, 4, 4, 4, 4]


def test_device_synthesis_matches_the_oracle_streams(gpu):
    """The device generator + quantizers reproduce the oracle's bytes (f64 transcendentals
    may differ in the last ulp, so a handful of blocks may differ by one code)."""
    nm = gpu
    n = 64 * 256
    for dtype in (nm.Q4_K, nm.Q8_0):
        buf = nm.DeviceBuffer(O.row_bytes(dtype, n))
        nm.lib().naiwa_synth(dtype, 77, 512, n, 0.0, 0.02, buf.ptr, 0)
        nm.synchronize()
        got = buf.download(np.uint8)
        want = O.quantize(dtype, O.normal(77, n, 0.0, 0.02, offset=512))
        bs = 144 if dtype == nm.Q4_K else 34
        same = (got.reshape(-1, bs) == want.reshape(-1, bs)).all(axis=1).mean()
        assert same >= 0.99, (dtype, same)
    buf = nm.DeviceBuffer(n * 4)
    nm.lib().naiwa_synth(nm.F32, 78, 0, n, 1.0, 2.0, buf.ptr, 0)
    nm.synchronize()
    got = buf.download(np.float32)
    want = O.normal(78, n, 1.0, 2.0)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("rows,H,E,k,ld", [
    (512, 2048, 64, 6, 8),   # DeepSeek-V2-Lite chunk: 6 routed + 2 shared columns
    (20, 2048, 64, 6, 8),    # the few-row router
    (3, 1024, 8, 2, 2),      # ld == k: the plain layout
])
def test_router_rows_ld_apart(gpu, rows, H, E, k, ld):
    """naiwa_router_topk_ld writes each row's k ids and weights at [t ld, t ld + k) -- the same
    values as the packed call -- and leaves the other columns as they were."""
    nm = gpu
    x = S.activations_bf16(2300 + rows, rows, H)
    W = O.normal(S.stream(2301, 0), E * H, 0.0, 0.02).reshape(E, H).astype(np.float32)
    want_ids, want_w, _ = gpu_router(nm, x, W, k, O.ROUTE_SOFTMAX_TOPK)
    fill_ids = np.full((rows, ld), 0xA5A5A5A5, np.uint32)
    fill_w = np.full((rows, ld), -3.5, np.float32)
    ids_d, w_d = nm.DeviceBuffer.from_array(fill_ids), nm.DeviceBuffer.from_array(fill_w)
    nm.router_topk(nm.DeviceBuffer.from_array(x), nm.BF16, nm.DeviceBuffer.from_array(W), rows, H, E, k,
                   ids_d, w_d, mode=O.ROUTE_SOFTMAX_TOPK, ld=ld)
    nm.synchronize()
    ids, w = ids_d.download(np.uint32).reshape(rows, ld), w_d.download(np.float32).reshape(rows, ld)
    assert np.array_equal(ids[:, :k], want_ids)
    assert np.array_equal(w[:, :k].view(np.uint32), want_w.view(np.uint32))
    assert (ids[:, k:] == 0xA5A5A5A5).all() and (w[:, k:] == -3.5).all()
    want_oracle, _ = O.topk(O.router_logits(O.from_bf16(x), W), k, O.ROUTE_SOFTMAX_TOPK)
    assert np.array_equal(ids[:, :k], want_oracle)
