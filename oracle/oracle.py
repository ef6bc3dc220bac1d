"""ctypes front end of the CPU oracle (liboracle.so, built from naiwa_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the reference results or the timed CPU baseline.  The
product library (naiwa-rs_amd/) never imports this module.

The C sources restate naiwa-rs's CPU expert path (src/moe/stages/cpu_miss.rs),
router top-k rule (src/moe/cached_layer.rs:357-363) and gather grouping
(src/moe/stages/gpu.rs:100-133); see naiwa_oracle.h for the per-function
citations and pinning.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, BF16 = 0, 1, 8, 12, 30
ROUTE_SOFTMAX_TOPK_RENORM, ROUTE_TOPK_SOFTMAX, ROUTE_SOFTMAX_TOPK = 0, 1, 2
ROUTER_CHUNK = 8

_lib = None


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class Stack(C.Structure):
    _fields_ = [("base", C.c_void_p), ("e", C.c_int32), ("n", C.c_int32),
                ("k", C.c_int32), ("dtype", C.c_int32)]


class Layer(C.Structure):
    _fields_ = [("router", C.c_void_p), ("gate", Stack), ("up", Stack), ("down", Stack)]


def _declare(L: C.CDLL) -> None:
    vp, i64, i32, u64 = C.c_void_p, C.c_int64, C.c_int, C.c_uint64
    L.orc_fp16_to_f32.restype = C.c_float
    L.orc_fp16_to_f32.argtypes = [C.c_uint16]
    L.orc_f32_to_fp16.restype = C.c_uint16
    L.orc_f32_to_fp16.argtypes = [C.c_float]
    L.orc_bf16_to_f32.restype = C.c_float
    L.orc_bf16_to_f32.argtypes = [C.c_uint16]
    L.orc_f32_to_bf16.restype = C.c_uint16
    L.orc_f32_to_bf16.argtypes = [C.c_float]
    L.orc_f32_to_bf16_n.argtypes = [vp, i64, vp]
    L.orc_bf16_to_f32_n.argtypes = [vp, i64, vp]
    L.orc_row_bytes.restype = i64
    L.orc_row_bytes.argtypes = [i32, i64]
    for name in ("orc_quantize", "orc_dequantize", "orc_dequantize_f64"):
        getattr(L, name).restype = i32
        getattr(L, name).argtypes = [i32, vp, i64, vp]
    L.orc_fill_normal.argtypes = [u64, u64, i64, C.c_float, C.c_float, vp]
    L.orc_vec_dot.restype = C.c_float
    L.orc_vec_dot.argtypes = [i32, vp, vp, i64]
    sp = C.POINTER(Stack)
    L.orc_fused_moe_decode.restype = i32
    L.orc_fused_moe_decode.argtypes = [sp, sp, sp, vp, vp, vp, i32, i32, vp]
    L.orc_fused_moe_decode_f64.restype = i32
    L.orc_fused_moe_decode_f64.argtypes = [sp, sp, sp, vp, vp, vp, i32, i32, vp]
    L.orc_router_logits.restype = i32
    L.orc_router_logits.argtypes = [vp, vp, i32, i32, i32, vp]
    L.orc_topk.restype = i32
    L.orc_topk.argtypes = [vp, i32, i32, i32, i32, vp, vp]
    L.orc_gather.restype = i32
    L.orc_gather.argtypes = [vp, i32, i32, vp, vp]
    L.orc_stack_decode.restype = i32
    L.orc_stack_decode.argtypes = [C.POINTER(Layer), i32, vp, i32, i32, i32, i32, i32, vp, vp]
    L.orc_stack_decode_mt.restype = i32
    L.orc_stack_decode_mt.argtypes = [C.POINTER(Layer), i32, vp, i32, i32, i32, i32, i32, vp, vp, i32]
    L.orc_fused_moe_decode_mt.restype = i32
    L.orc_fused_moe_decode_mt.argtypes = [sp, sp, sp, vp, vp, vp, i32, i32, vp, i32]


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ---- conversions ----------------------------------------------------------------

def to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(_p(x), x.size, _p(out))
    return out


def from_bf16(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_n(_p(h), h.size, _p(out))
    return out


def fp16_to_f32(h: int) -> float:
    return lib().orc_fp16_to_f32(h)


def f32_to_fp16(f: float) -> int:
    return lib().orc_f32_to_fp16(f)


# ---- formats --------------------------------------------------------------------

def row_bytes(dtype: int, k: int) -> int:
    return lib().orc_row_bytes(dtype, k)


def quantize(dtype: int, x: np.ndarray) -> np.ndarray:
    """Quantize the last axis of x (f32) row by row; returns uint8 [..., row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    rb = row_bytes(dtype, k)
    if rb < 0:
        raise ValueError(f"K={k} not a multiple of the block size of dtype {dtype}")
    out = np.empty(x.shape[:-1] + (rb,), dtype=np.uint8)
    if lib().orc_quantize(dtype, _p(x), x.size, _p(out)) != 0:
        raise ValueError("quantize failed")
    return out


def dequantize(dtype: int, q: np.ndarray, k: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rb = row_bytes(dtype, k)
    rows = q.size // rb
    out = np.empty(q.shape[:-1] + (k,), dtype=np.float32)
    if lib().orc_dequantize(dtype, _p(q), rows * k, _p(out)) != 0:
        raise ValueError("dequantize failed")
    return out


def dequantize_f64(dtype: int, q: np.ndarray, k: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rb = row_bytes(dtype, k)
    rows = q.size // rb
    out = np.empty(q.shape[:-1] + (k,), dtype=np.float64)
    if lib().orc_dequantize_f64(dtype, _p(q), rows * k, _p(out)) != 0:
        raise ValueError("dequantize failed")
    return out


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0, offset: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(seed, offset, n, mean, std, _p(out))
    return out


def vec_dot(dtype: int, row: np.ndarray, x: np.ndarray) -> float:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().orc_vec_dot(dtype, _p(row), _p(x), x.size)


# ---- expert path ----------------------------------------------------------------

def stack(q: np.ndarray, dtype: int, n: int, k: int) -> Stack:
    """q: uint8 [E, N, row_bytes] stacked expert bytes (kept alive by the caller)."""
    assert q.dtype == np.uint8 and q.flags["C_CONTIGUOUS"]
    e = q.shape[0]
    assert q.size == e * n * row_bytes(dtype, k)
    return Stack(q.ctypes.data, e, n, k, dtype)


def fused_moe_decode(gate: Stack, up: Stack, down: Stack, xs: np.ndarray, ids: np.ndarray,
                     w: np.ndarray) -> np.ndarray:
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, width = ids.shape
    out = np.empty((rows, gate.k), dtype=np.float32)
    rc = lib().orc_fused_moe_decode(C.byref(gate), C.byref(up), C.byref(down), _p(xs), _p(ids),
                                    _p(w), rows, width, _p(out))
    if rc != 0:
        raise ValueError(f"orc_fused_moe_decode failed ({rc})")
    return out


def fused_moe_decode_mt(gate: Stack, up: Stack, down: Stack, xs: np.ndarray, ids: np.ndarray,
                        w: np.ndarray, threads: int) -> np.ndarray:
    """fused_moe_decode on `threads` host threads (bit-identical; the CPU baseline)."""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, width = ids.shape
    out = np.empty((rows, gate.k), dtype=np.float32)
    rc = lib().orc_fused_moe_decode_mt(C.byref(gate), C.byref(up), C.byref(down), _p(xs), _p(ids),
                                       _p(w), rows, width, _p(out), threads)
    if rc != 0:
        raise ValueError(f"orc_fused_moe_decode_mt failed ({rc})")
    return out


def fused_moe_decode_f64(gate: Stack, up: Stack, down: Stack, xs: np.ndarray, ids: np.ndarray,
                         w: np.ndarray) -> np.ndarray:
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, width = ids.shape
    out = np.empty((rows, gate.k), dtype=np.float64)
    rc = lib().orc_fused_moe_decode_f64(C.byref(gate), C.byref(up), C.byref(down), _p(xs),
                                        _p(ids), _p(w), rows, width, _p(out))
    if rc != 0:
        raise ValueError(f"orc_fused_moe_decode_f64 failed ({rc})")
    return out


def router_logits(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    rows, H = x.shape
    E = W.shape[0]
    out = np.empty((rows, E), dtype=np.float32)
    if lib().orc_router_logits(_p(x), _p(W), rows, H, E, _p(out)) != 0:
        raise ValueError("router_logits failed")
    return out


def topk(logits: np.ndarray, k: int, mode: int = ROUTE_SOFTMAX_TOPK_RENORM):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, E = logits.shape
    ids = np.empty((rows, k), dtype=np.uint32)
    w = np.empty((rows, k), dtype=np.float32)
    if lib().orc_topk(_p(logits), rows, E, k, mode, _p(ids), _p(w)) != 0:
        raise ValueError("topk failed")
    return ids, w


def gather(ids: np.ndarray, E: int):
    ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
    perm = np.empty(ids.size, dtype=np.uint32)
    offsets = np.empty(E + 1, dtype=np.uint32)
    if lib().orc_gather(_p(ids), ids.size, E, _p(perm), _p(offsets)) != 0:
        raise ValueError("gather failed")
    return perm, offsets


def stack_decode(layers: list, x_bf16: np.ndarray, E: int, k: int,
                 mode: int = ROUTE_SOFTMAX_TOPK_RENORM, threads: int = 0):
    """layers: list of (router f32 [E,H], (gate_q, up_q, down_q), (dtype_g, dtype_u, dtype_d), I).
    threads > 0 runs the expert path on that many host threads (bit-identical).

    Returns (x_out bf16 [rows,H], ids [L,rows,k], w [L,rows,k])."""
    x = np.array(x_bf16, dtype=np.uint16, copy=True, order="C")
    rows, H = x.shape
    arr = (Layer * len(layers))()
    keep = []
    for i, (router, (gq, uq, dq), (dg, du, dd), inter) in enumerate(layers):
        router = np.ascontiguousarray(router, dtype=np.float32)
        keep.append(router)
        arr[i].router = router.ctypes.data
        arr[i].gate = stack(gq, dg, inter, H)
        arr[i].up = stack(uq, du, inter, H)
        arr[i].down = stack(dq, dd, H, inter)
    ids = np.empty((len(layers), rows, k), dtype=np.uint32)
    w = np.empty((len(layers), rows, k), dtype=np.float32)
    if threads > 0:
        rc = lib().orc_stack_decode_mt(arr, len(layers), _p(x), rows, H, E, k, mode, _p(ids), _p(w), threads)
    else:
        rc = lib().orc_stack_decode(arr, len(layers), _p(x), rows, H, E, k, mode, _p(ids), _p(w))
    if rc != 0:
        raise ValueError(f"orc_stack_decode failed ({rc})")
    return x, ids, w
