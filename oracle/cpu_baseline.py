"""ctypes front end of the CPU baseline (libcpubase.so, built from cpu_baseline.c).

TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it and tests/ check
it; the product library never imports this module.  It restates the reference's
CPU expert path (fused_moe_decode, src/moe/stages/cpu_miss.rs:13-20) with int8
activations and AVX2 integer dots on a persistent thread pool, so its results
differ from the oracle's f32 path by the activation rounding.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

from oracle import Stack

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcpubase.so")

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-s", "-C", HERE, "libcpubase.so"], check=True)
        L = C.CDLL(LIB_PATH)
        L.cb_pool_create.restype = C.c_void_p
        L.cb_pool_create.argtypes = [C.c_int]
        L.cb_pool_destroy.restype = None
        L.cb_pool_destroy.argtypes = [C.c_void_p]
        L.cb_threads.restype = C.c_int
        L.cb_threads.argtypes = [C.c_void_p]
        L.cb_fused_moe_decode.restype = C.c_int
        L.cb_fused_moe_decode.argtypes = [C.c_void_p, C.POINTER(Stack), C.POINTER(Stack), C.POINTER(Stack),
                                          C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
        _lib = L
    return _lib


def physical_cores() -> int | None:
    """Physical cores of this host from lscpu (distinct (core, socket) pairs), or None."""
    try:
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, check=True).stdout
    except (OSError, subprocess.CalledProcessError):
        return None
    pairs = {line.strip() for line in out.splitlines() if line and not line.startswith("#")}
    return len(pairs) or None


class Pool:
    """A persistent pool of `threads` host threads (the calling thread included)."""

    def __init__(self, threads: int):
        self._h = lib().cb_pool_create(threads)
        if not self._h:
            raise MemoryError("cb_pool_create failed")
        self.threads = lib().cb_threads(self._h)

    def close(self) -> None:
        if self._h:
            lib().cb_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def fused_moe_decode(self, gate: Stack, up: Stack, down: Stack, xs: np.ndarray, ids: np.ndarray,
                         w: np.ndarray) -> np.ndarray:
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        rows, width = ids.shape
        out = np.empty((rows, gate.k), dtype=np.float32)
        rc = lib().cb_fused_moe_decode(self._h, C.byref(gate), C.byref(up), C.byref(down), xs.ctypes.data,
                                       ids.ctypes.data, w.ctypes.data, rows, width, out.ctypes.data)
        if rc != 0:
            raise ValueError(f"cb_fused_moe_decode failed ({rc})")
        return out
