"""The allocation-free decode entry point (naiwa_moe_decode_noalloc), called
through the C ABI: on two calls in a row -- the second with a smaller input --
its output is bit-identical to naiwa_moe_decode_ex's on the same inputs (both
run the same kernels; only the scratch differs) and within the 1e-2 bar of the
oracle.  An accumulating call and a request past the fixed scratch are checked
too.  This is the last test file collected, so a failure here hides nothing."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
import synthetic as S

pytestmark = pytest.mark.gpu
TOL = 1e-2
DECODE_ACCUMULATE = 1   # NAIWA_DECODE_ACCUMULATE


def _decode(nm, fn, banks, xd, ids_d, w_d, rows, k, out, flags=0):
    g, u, d = banks.gate.desc(), banks.up.desc(), banks.down.desc()
    return getattr(nm.lib(), fn)(C.byref(g), C.byref(u), C.byref(d), xd.ptr, nm.BF16, ids_d.ptr, w_d.ptr, rows, k,
                                 nm.ACT_SILU, out.ptr, flags, 0)


def test_noalloc_matches_the_allocating_entry_point(gpu):
    nm = gpu
    E, H, I, k = 128, 2048, 768, 8
    dt = (O.Q4_K,) * 3
    g, u, d, r = S.layer(7000, E, H, I, dt)
    banks = nm.LayerBanks(E, H, I, dt)
    for e in range(E):
        banks.load(e, g[e], u[e], d[e])
    stacks = (O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I))
    keep = []
    for call, rows in enumerate((8, 3)):
        x = S.activations_bf16(7001 + call, rows, H)
        ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k, O.ROUTE_SOFTMAX_TOPK_RENORM)
        xd = nm.DeviceBuffer.from_array(x)
        ids_d = nm.DeviceBuffer.from_array(ids.astype(np.uint32))
        w_d = nm.DeviceBuffer.from_array(w.astype(np.float32))
        ref, got = nm.DeviceBuffer(rows * H * 4), nm.DeviceBuffer(rows * H * 4)
        keep += [xd, ids_d, w_d, ref, got]
        print(f"[noalloc call {call} rows={rows}]", flush=True)
        assert _decode(nm, "naiwa_moe_decode_ex", banks, xd, ids_d, w_d, rows, k, ref) == 0
        assert _decode(nm, "naiwa_moe_decode_noalloc", banks, xd, ids_d, w_d, rows, k, got) == 0
        nm.synchronize()
        a = ref.download(np.float32).reshape(rows, H)
        b = got.download(np.float32).reshape(rows, H)
        assert np.array_equal(a, b), call
        want = O.fused_moe_decode(*stacks, O.from_bf16(x), ids, w)
        err = S.max_rel_err(b, want)
        print(f"  bit-identical, max_rel_err={err:.3e}", flush=True)
        assert err < TOL
    # an accumulating call continues from out's values, as the allocating one does
    rows = 2
    x = S.activations_bf16(7010, rows, H)
    ids, w = O.topk(O.router_logits(O.from_bf16(x), r), k, O.ROUTE_SOFTMAX_TOPK_RENORM)
    xd = nm.DeviceBuffer.from_array(x)
    ids_d = nm.DeviceBuffer.from_array(ids.astype(np.uint32))
    w_d = nm.DeviceBuffer.from_array(w.astype(np.float32))
    start = np.linspace(-1, 1, rows * H, dtype=np.float32)
    ref, got = nm.DeviceBuffer.from_array(start), nm.DeviceBuffer.from_array(start)
    assert _decode(nm, "naiwa_moe_decode_ex", banks, xd, ids_d, w_d, rows, k, ref, DECODE_ACCUMULATE) == 0
    assert _decode(nm, "naiwa_moe_decode_noalloc", banks, xd, ids_d, w_d, rows, k, got, DECODE_ACCUMULATE) == 0
    nm.synchronize()
    assert np.array_equal(ref.download(np.float32), got.download(np.float32))


def test_noalloc_rejects_requests_past_its_scratch(gpu):
    nm = gpu
    H, I, k = 256, 14336, 2
    dt = (O.Q8_0,) * 3
    banks = nm.LayerBanks(2, H, I, dt)
    rows = 128    # 256 pairs: h (30 KB a pair) and the K parts' dots pass the 8 MiB array
    xd = nm.DeviceBuffer(rows * H * 2)
    ids_d = nm.DeviceBuffer.from_array(np.zeros((rows, k), np.uint32))
    w_d = nm.DeviceBuffer.from_array(np.zeros((rows, k), np.float32))
    out = nm.DeviceBuffer(rows * H * 4)
    assert _decode(nm, "naiwa_moe_decode_noalloc", banks, xd, ids_d, w_d, rows, k, out) == nm.E_TOO_LARGE
