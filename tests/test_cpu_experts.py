"""The product CPU expert path (naiwa_cpu_moe_decode, the reference's fused_moe_decode
contract, src/moe/stages/cpu_miss.rs:13-20) against the oracle on the same bytes.
Host only: the library's CPU path touches no device."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
import synthetic as S
from naiwa_moe import policy as P
from naiwa_moe._lib import E_BAD_ID, HostExperts, NaiwaError, lib

TOL = 1e-4  # f32 on both sides; only the summation order differs


def oracle(g, u, d, dt, H, I, xs, ids, w):
    gs, us, ds = O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I)
    return O.fused_moe_decode(gs, us, ds, xs, ids, w)


@pytest.mark.parametrize("H,I,E,dt,rows,width", [
    (1024, 2048, 8, (O.Q8_0,) * 3, 1, 2),                    # C1: Mixtral-style layer, Q8_0
    (512, 256, 8, (O.Q4_K,) * 3, 3, 4),                      # Q4_K, several rows
    (512, 288, 6, (O.Q4_K, O.Q4_K, O.Q8_0), 2, 3),           # DS-V2-Lite style: Q8_0 down
])
def test_cpu_decode_matches_the_oracle(H, I, E, dt, rows, width):
    g, u, d, _ = S.layer(2400 + H, E, H, I, dt)
    xs = O.from_bf16(S.activations_bf16(2401 + H, rows, H)).astype(np.float32)
    rng = np.random.default_rng(H)
    ids = np.stack([rng.choice(E, size=width, replace=False) for _ in range(rows)]).astype(np.uint32)
    w = rng.random((rows, width)).astype(np.float32)
    if width > 2:
        w[0, -1] = 0.0                       # a padding entry (reference cpu_miss.rs:90-100)
    got = P.cpu_moe_decode(g, u, d, dt, H, I, xs, ids, w)
    want = oracle(g, u, d, dt, H, I, xs, ids, w)
    assert S.max_rel_err(got, want) < TOL


def test_cpu_decode_gelu_and_interleaved_stacks():
    """GELU (tanh) activation, and host stacks with each expert's gate | up | down
    adjacent under one stride (the staged-upload layout)."""
    H, I, E, rows, width = 512, 256, 5, 2, 2
    dt = (O.Q4_K,) * 3
    g, u, d, _ = S.layer(2450, E, H, I, dt)
    gb, ub, db = g.reshape(E, -1), u.reshape(E, -1), d.reshape(E, -1)
    stride = gb.shape[1] + ub.shape[1] + db.shape[1] + 64
    blob = np.zeros((E, stride), dtype=np.uint8)
    blob[:, :gb.shape[1]] = gb
    blob[:, gb.shape[1]:gb.shape[1] + ub.shape[1]] = ub
    blob[:, gb.shape[1] + ub.shape[1]:gb.shape[1] + ub.shape[1] + db.shape[1]] = db
    base = blob.ctypes.data
    ex = HostExperts(base, base + gb.shape[1], base + gb.shape[1] + ub.shape[1], stride, stride, stride,
                     dt[0], dt[1], dt[2], E, H, I)
    xs = O.from_bf16(S.activations_bf16(2451, rows, H)).astype(np.float32)
    ids = np.array([[4, 1], [0, 4]], dtype=np.uint32)
    w = np.array([[0.7, 0.3], [0.5, 0.5]], dtype=np.float32)
    out = np.empty((rows, H), dtype=np.float32)
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)
    ACT_GELU = 1
    assert lib().naiwa_cpu_moe_decode(C.byref(ex), ptr(xs), ptr(ids), ptr(w), rows, width, ACT_GELU, ptr(out)) == 0
    # GELU(tanh) against an fp64 numpy restatement (the oracle's fused path is SiLU only,
    # as the reference's is)
    G = O.dequantize_f64(dt[0], g, H).reshape(E, I, H)
    U = O.dequantize_f64(dt[1], u, H).reshape(E, I, H)
    D = O.dequantize_f64(dt[2], d, I).reshape(E, H, I)
    want = np.zeros((rows, H))
    for t in range(rows):
        x64 = xs[t].astype(np.float64)
        for j in range(width):
            e = ids[t, j]
            gx = G[e] @ x64
            gel = 0.5 * gx * (1 + np.tanh(np.sqrt(2 / np.pi) * (gx + 0.044715 * gx ** 3)))
            want[t] += w[t, j] * (D[e] @ (gel * (U[e] @ x64)))
    assert S.max_rel_err(out, want) < TOL
    # and the SiLU path over the same interleaved stacks agrees with the oracle
    assert lib().naiwa_cpu_moe_decode(C.byref(ex), ptr(xs), ptr(ids), ptr(w), rows, width, 0, ptr(out)) == 0
    gs, us, ds = O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I)
    assert S.max_rel_err(out, O.fused_moe_decode(gs, us, ds, xs, ids, w)) < TOL


def test_cpu_decode_rejects_bad_ids():
    H, I, E = 256, 256, 4
    dt = (O.Q4_K,) * 3
    g, u, d, _ = S.layer(2460, E, H, I, dt)
    xs = np.ones((1, H), np.float32)
    with pytest.raises(NaiwaError) as e:
        P.cpu_moe_decode(g, u, d, dt, H, I, xs, np.array([[1, 4]], np.uint32), np.ones((1, 2), np.float32))
    assert e.value.rc == E_BAD_ID
