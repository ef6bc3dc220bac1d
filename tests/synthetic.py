"""Seeded synthetic inputs for the parity tests (host side, from the oracle's
counter-based generator), shaped like the benchmark configurations.

Stream ids: every tensor draws its values from stream (seed * 64 + tensor_id),
so a layer's tensors never share values and any test can regenerate them."""
from __future__ import annotations

import numpy as np

import oracle as O

T_GATE, T_UP, T_DOWN, T_ROUTER, T_X = 0, 1, 2, 3, 4


def stream(seed: int, tensor: int) -> int:
    return seed * 64 + tensor


_POOL = None


def _pool():
    global _POOL
    if _POOL is None:
        import concurrent.futures as cf
        import os
        _POOL = cf.ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1))
    return _POOL


def quantized_stack(seed: int, tensor: int, E: int, N: int, K: int, dtype: int,
                    std: float = 0.02) -> np.ndarray:
    """uint8 [E, N, row_bytes]: N(0, std) values quantized row by row.  Experts are
    generated and quantized in parallel (the counter-based stream at each expert's
    offset gives the same values as one sequential draw)."""
    out = np.empty((E, N, O.row_bytes(dtype, K)), dtype=np.uint8)

    def one(e):
        vals = O.normal(stream(seed, tensor), N * K, 0.0, std, offset=e * N * K)
        out[e] = O.quantize(dtype, vals.reshape(N, K))

    list(_pool().map(one, range(E)))
    return out


def layer(seed: int, E: int, H: int, I: int, dtypes=(O.Q4_K, O.Q4_K, O.Q4_K), std: float = 0.02):
    """(gate [E,I,rb], up [E,I,rb], down [E,H,rb], router f32 [E,H])."""
    g = quantized_stack(seed, T_GATE, E, I, H, dtypes[0], std)
    u = quantized_stack(seed, T_UP, E, I, H, dtypes[1], std)
    d = quantized_stack(seed, T_DOWN, E, H, I, dtypes[2], std)
    r = O.normal(stream(seed, T_ROUTER), E * H, 0.0, 0.02).reshape(E, H)
    return g, u, d, r


def activations_bf16(seed: int, rows: int, H: int) -> np.ndarray:
    return O.to_bf16(O.normal(stream(seed, T_X), rows * H).reshape(rows, H))


def max_rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max |want| over the whole output (norm-relative)."""
    want = np.asarray(want, dtype=np.float64)
    den = np.abs(want).max()
    return float(np.abs(np.asarray(got, dtype=np.float64) - want).max() / (den if den > 0 else 1.0))
