"""GGUF checkpoints (include/naiwa_gguf.h): a read-only mapping of the file, its
tensors and metadata, and one layer's stacked routed-expert projections
blk.<layer>.ffn_{gate,up,down}_exps.weight ([E, N, K]; expert e is
expert_range(e), src/moe/expert.rs:123-145), copied into pinned host stacks for
expert uploads.  The reference reads the same files through the fork's GGUF
loader (src/load.rs:414-452)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib
from .ops import BLOCK, HostExpertStacks

PROJ_GATE, PROJ_UP, PROJ_DOWN = 0, 1, 2


class GgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_int), ("dims", C.c_int64 * 4), ("dtype", C.c_int),
                ("offset", C.c_uint64), ("bytes", C.c_uint64), ("data", C.c_void_p)]


class ExpertStack(C.Structure):
    _fields_ = [("data", C.c_void_p), ("experts", C.c_int), ("n", C.c_int), ("k", C.c_int), ("dtype", C.c_int),
                ("expert_bytes", C.c_uint64)]


def type_size(dtype: int) -> tuple[int, int]:
    """(block values, block bytes) of a GGML type id; (0, 0) when unknown."""
    b, n = C.c_int(), C.c_int()
    check(lib().naiwa_ggml_type_size(dtype, C.byref(b), C.byref(n)), "naiwa_ggml_type_size")
    return b.value, n.value


def _view(ptr: int, nbytes: int) -> np.ndarray:
    """uint8 view of mapped (read-only) bytes; valid while the file is open."""
    if nbytes == 0:
        return np.empty(0, dtype=np.uint8)
    buf = (C.c_uint8 * nbytes).from_address(ptr)
    arr = np.frombuffer(buf, dtype=np.uint8)
    arr.flags.writeable = False
    return arr


class GgufFile:
    """An open GGUF file.  Views returned by tensor_bytes / expert_view stay valid
    until close()."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().naiwa_gguf_open(str(path).encode(), C.byref(h)), f"naiwa_gguf_open({path})")
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            lib().naiwa_gguf_close(self._h)
            self._h = C.c_void_p()

    __del__ = close

    def __enter__(self) -> "GgufFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    @property
    def version(self) -> int:
        v = C.c_uint32()
        check(lib().naiwa_gguf_version(self._h, C.byref(v)), "naiwa_gguf_version")
        return v.value

    @property
    def alignment(self) -> int:
        v = C.c_uint64()
        check(lib().naiwa_gguf_alignment(self._h, C.byref(v)), "naiwa_gguf_alignment")
        return v.value

    def tensors(self) -> list[GgufTensor]:
        n = C.c_int()
        check(lib().naiwa_gguf_tensor_count(self._h, C.byref(n)), "naiwa_gguf_tensor_count")
        out = []
        for i in range(n.value):
            t = GgufTensor()
            check(lib().naiwa_gguf_tensor_at(self._h, i, C.byref(t)), "naiwa_gguf_tensor_at")
            out.append(t)
        return out

    def find(self, name: str) -> GgufTensor | None:
        t = GgufTensor()
        rc = lib().naiwa_gguf_find(self._h, name.encode(), C.byref(t))
        if rc == -6:  # NAIWA_E_NOT_FOUND
            return None
        check(rc, f"naiwa_gguf_find({name})")
        return t

    def tensor_bytes(self, name: str) -> np.ndarray:
        t = self.find(name)
        if t is None:
            raise KeyError(name)
        if not t.bytes:
            raise ValueError(f"{name}: type {t.dtype} has no known block size")
        return _view(t.data, t.bytes)

    def meta_u64(self, key: str) -> int | None:
        v = C.c_uint64()
        rc = lib().naiwa_gguf_meta_u64(self._h, key.encode(), C.byref(v))
        if rc == -6:
            return None
        check(rc, f"naiwa_gguf_meta_u64({key})")
        return v.value

    def meta_str(self, key: str) -> str | None:
        n = C.c_int()
        rc = lib().naiwa_gguf_meta_string(self._h, key.encode(), None, 0, C.byref(n))
        if rc == -6:
            return None
        if rc not in (0, -1):  # -1: the length probe with no buffer
            check(rc, f"naiwa_gguf_meta_string({key})")
        buf = C.create_string_buffer(n.value + 1)
        check(lib().naiwa_gguf_meta_string(self._h, key.encode(), buf, n.value + 1, C.byref(n)),
              f"naiwa_gguf_meta_string({key})")
        return buf.raw[: n.value].decode("utf-8", errors="replace")

    def expert_stack(self, layer: int, proj: int) -> ExpertStack:
        s = ExpertStack()
        check(lib().naiwa_gguf_expert_stack(self._h, layer, proj, C.byref(s)), "naiwa_gguf_expert_stack")
        return s

    def expert_view(self, layer: int, proj: int) -> np.ndarray:
        """[E, expert_bytes] uint8 view of a layer's stacked projection."""
        s = self.expert_stack(layer, proj)
        return _view(s.data, s.experts * s.expert_bytes).reshape(s.experts, s.expert_bytes)

    def host_stacks(self, layer: int) -> HostExpertStacks:
        """Pinned host copies of a layer's three projections (gate/up [E, I, H], down
        [E, H, I]), the sources of expert uploads."""
        g, u, d = (self.expert_stack(layer, p) for p in (PROJ_GATE, PROJ_UP, PROJ_DOWN))
        if not (g.experts == u.experts == d.experts and (g.n, g.k) == (u.n, u.k) == (d.k, d.n)):
            raise ValueError(f"layer {layer}: expert stacks disagree: gate [{g.experts},{g.n},{g.k}], "
                             f"up [{u.experts},{u.n},{u.k}], down [{d.experts},{d.n},{d.k}]")
        for p, s in enumerate((g, u, d)):
            if s.dtype not in BLOCK:
                raise ValueError(f"layer {layer}: projection {p} is GGML type {s.dtype}, which is not served")
        stacks = HostExpertStacks(g.experts, g.k, g.n, (g.dtype, u.dtype, d.dtype))
        for p, s in enumerate((g, u, d)):
            if stacks.expert_bytes[p] != s.expert_bytes:
                raise ValueError(f"layer {layer}: projection {p} of type {s.dtype} is not served")
            np.copyto(stacks.view(p), self.expert_view(layer, p))
        return stacks
