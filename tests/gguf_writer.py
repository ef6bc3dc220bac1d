"""A small GGUF writer for the tests (the public file layout): header "GGUF",
version, tensor count, metadata count; metadata key/type/value; tensor infos
(name, n_dims, dims ne0.., type, offset); data at the next multiple of the
alignment, each tensor at an aligned offset.  All little-endian."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}


def _string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STRING:
        return _string(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_SCALAR[t], v)


def gguf_bytes(metadata: list[tuple[str, int, object]], tensors: list[tuple[str, tuple[int, ...], int, bytes]],
               version: int = 3, alignment: int = 32) -> bytes:
    """metadata: (key, type, value) (an ARRAY value is (element type, items));
    tensors: (name, dims ne0 first, GGML type, raw bytes)."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata))
    meta = b"".join(_string(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in metadata)
    infos, offsets, off = [], [], 0
    for name, dims, dtype, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        infos.append(_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                     + struct.pack("<IQ", dtype, off))
        off += len(data)
    body = head + meta + b"".join(infos)
    pad = (-len(body)) % alignment
    out = bytearray(body + b"\0" * pad)
    base = len(out)
    for (name, dims, dtype, data), o in zip(tensors, offsets):
        out += b"\0" * (base + o - len(out))
        out += data
    return bytes(out)


def write_gguf(path, metadata, tensors, version: int = 3, alignment: int = 32) -> None:
    with open(path, "wb") as f:
        f.write(gguf_bytes(metadata, tensors, version, alignment))


def expert_tensors(layer: int, g: np.ndarray, u: np.ndarray, d: np.ndarray, router: np.ndarray,
                   H: int, I: int, dtypes: tuple[int, int, int]) -> list:
    """One MoE layer's tensors as the checkpoints name them: stacked experts
    [E, N, K] (dims ne0 = K first) and the f32 router [E, H]."""
    E = g.shape[0]
    return [
        (f"blk.{layer}.ffn_gate_inp.weight", (H, E), 0, np.ascontiguousarray(router, dtype=np.float32).tobytes()),
        (f"blk.{layer}.ffn_gate_exps.weight", (H, I, E), dtypes[0], g.tobytes()),
        (f"blk.{layer}.ffn_up_exps.weight", (H, I, E), dtypes[1], u.tobytes()),
        (f"blk.{layer}.ffn_down_exps.weight", (I, H, E), dtypes[2], d.tobytes()),
    ]
