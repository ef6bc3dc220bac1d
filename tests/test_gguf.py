"""The GGUF reader (include/naiwa_gguf.h) on files written by tests/gguf_writer.py:
tensors, metadata and per-expert slices round-trip byte for byte; the
reference's own retyping cases (src/load.rs:516-558: a Q4_0 tensor retyped to
IQ4_NL is readable, to a retired id it is not); malformed files fail with
NAIWA_E_FORMAT instead of reading outside the file."""
import struct

import numpy as np
import pytest

import naiwa_moe as nm
import oracle as O
import synthetic as S
from gguf_writer import ARRAY, BOOL, F32, I64, STRING, U32, U8, expert_tensors, gguf_bytes, write_gguf
from naiwa_moe.gguf import PROJ_DOWN, PROJ_GATE, PROJ_UP, GgufFile, type_size

H, I, E = 256, 64, 4
DT = (O.Q4_K, O.Q4_K, O.Q8_0)


def _layer(seed):
    g, u, d, r = S.layer(seed, E, H, I, DT)
    return g, u, d, r


def _meta():
    return [("general.architecture", STRING, "qwen3moe"),
            ("qwen3moe.expert_count", U32, E),
            ("qwen3moe.expert_used_count", U32, 2),
            ("general.file_type", U8, 15),
            ("general.quantized", BOOL, True),
            ("qwen3moe.rope.freq_base", F32, 1e6),
            ("general.size", I64, 12345),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, ["a", "bc", "def"])),
            ("qwen3moe.layer_sizes", ARRAY, (U32, [1, 2, 3]))]


@pytest.fixture(scope="module")
def two_layers(tmp_path_factory):
    layers = [_layer(300), _layer(301)]
    tensors = []
    for l, (g, u, d, r) in enumerate(layers):
        tensors += expert_tensors(l, g, u, d, r, H, I, DT)
    path = tmp_path_factory.mktemp("gguf") / "model.gguf"
    write_gguf(path, _meta(), tensors)
    return path, layers, tensors


def test_tensors_and_metadata_round_trip(two_layers):
    path, layers, tensors = two_layers
    with GgufFile(path) as f:
        assert f.version == 3 and f.alignment == 32
        got = f.tensors()
        assert [t.name.decode() for t in got] == [t[0] for t in tensors]
        for t, (name, dims, dtype, data) in zip(got, tensors):
            assert t.n_dims == len(dims) and tuple(t.dims[: t.n_dims]) == dims and t.dtype == dtype
            assert t.bytes == len(data) and t.offset % 32 == 0
            assert f.tensor_bytes(name).tobytes() == data
        assert f.meta_str("general.architecture") == "qwen3moe"
        assert f.meta_u64("qwen3moe.expert_count") == E and f.meta_u64("general.file_type") == 15
        assert f.meta_u64("general.quantized") == 1 and f.meta_u64("general.size") == 12345
        assert f.meta_u64("no.such.key") is None and f.find("no.such.tensor") is None
        with pytest.raises(nm.NaiwaError):
            f.meta_u64("general.architecture")  # a string
        with pytest.raises(nm.NaiwaError):
            f.meta_str("qwen3moe.expert_count")  # an integer


def test_expert_slices_follow_expert_range(two_layers):
    path, layers, _ = two_layers
    with GgufFile(path) as f:
        for l, (g, u, d, r) in enumerate(layers):
            for p, (stack, n, k, dt) in enumerate(((g, I, H, DT[0]), (u, I, H, DT[1]), (d, H, I, DT[2]))):
                s = f.expert_stack(l, p)
                assert (s.experts, s.n, s.k, s.dtype) == (E, n, k, dt)
                assert s.expert_bytes == n * nm.row_bytes(dt, k)
                view = f.expert_view(l, p)
                flat = stack.reshape(-1)
                for e in range(E):
                    rg = nm.expert_range(dt, n, k, e)
                    assert view[e].tobytes() == flat[rg.start:rg.stop].tobytes()
            router = f.tensor_bytes(f"blk.{l}.ffn_gate_inp.weight").view(np.float32).reshape(E, H)
            assert np.array_equal(router, r)
        with pytest.raises(nm.NaiwaError):
            f.expert_stack(2, PROJ_GATE)  # no such layer
        with pytest.raises(nm.NaiwaError):
            f.expert_stack(0, 3)


def test_type_sizes_match_the_block_formats():
    assert type_size(O.Q4_K) == (256, 144) and type_size(O.Q8_0) == (32, 34)
    assert type_size(0) == (1, 4) and type_size(30) == (1, 2)   # F32, BF16
    assert type_size(2) == (32, 18) and type_size(20) == (32, 18)  # Q4_0, IQ4_NL (src/load.rs:517-518)
    assert type_size(4) == (0, 0)  # a retired id


def _retyped(tmp_path, dtype):
    """src/load.rs:519-541: a Q4_0 [2, 32] tensor named blk.0.ffn_down_exps.weight,
    its type id patched after the name, n_dims (u32) and dims (2 x u64)."""
    data = bytes(2 * 18)
    raw = bytearray(gguf_bytes([("general.architecture", STRING, "qwen4exp")],
                               [("blk.0.ffn_down_exps.weight", (32, 2), 2, data)]))
    name = b"blk.0.ffn_down_exps.weight"
    at = raw.find(name) + len(name) + 4 + 2 * 8
    assert struct.unpack_from("<I", raw, at)[0] == 2
    struct.pack_into("<I", raw, at, dtype)
    path = tmp_path / f"t{dtype}.gguf"
    path.write_bytes(bytes(raw))
    return path


def test_retyped_tensors(tmp_path):
    with GgufFile(_retyped(tmp_path, 20)) as f:  # IQ4_NL: same block layout, readable
        t = f.find("blk.0.ffn_down_exps.weight")
        assert t.dtype == 20 and t.bytes == 36
    with GgufFile(_retyped(tmp_path, 4)) as f:  # retired id: listed, not readable
        t = f.find("blk.0.ffn_down_exps.weight")
        assert t.dtype == 4 and t.bytes == 0 and not t.data
        with pytest.raises(ValueError):
            f.tensor_bytes("blk.0.ffn_down_exps.weight")
        with pytest.raises(nm.NaiwaError) as ei:
            f.expert_stack(0, PROJ_DOWN)
        assert ei.value.rc == nm.E_UNSUPPORTED


def test_version_2_and_other_alignments(tmp_path):
    g, u, d, r = _layer(302)
    tensors = expert_tensors(0, g, u, d, r, H, I, DT)
    for version, align in ((2, 32), (3, 64), (3, 256)):
        meta = [("general.alignment", U32, align)] if align != 32 else []
        path = tmp_path / f"v{version}a{align}.gguf"
        write_gguf(path, meta, tensors, version=version, alignment=align)
        with GgufFile(path) as f:
            assert f.version == version and f.alignment == align
            assert f.expert_view(0, PROJ_UP).tobytes() == u.tobytes()


def _rc_of_open(path):
    try:
        GgufFile(path).close()
        return 0
    except nm.NaiwaError as e:
        return e.rc


def test_malformed_files_are_rejected(tmp_path):
    g, u, d, r = _layer(303)
    good = gguf_bytes(_meta(), expert_tensors(0, g, u, d, r, H, I, DT))
    cases = {
        "magic": b"GGUX" + good[4:],
        "version1": good[:4] + struct.pack("<I", 1) + good[8:],
        "version4": good[:4] + struct.pack("<I", 4) + good[8:],
        "empty": b"",
        "header_only": good[:12],
        "cut_in_metadata": good[:60],
        "cut_in_data": good[:-100],
        "huge_count": good[:8] + struct.pack("<Q", 1 << 40) + good[16:],
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        assert _rc_of_open(p) == nm.E_FORMAT, name
    assert _rc_of_open(tmp_path / "missing.gguf") == nm.E_IO
    # a tensor offset that is not aligned, a duplicate name, 5 dims, an odd alignment
    t0 = ("a", (32,), 0, bytes(128))
    raw = bytearray(gguf_bytes([], [t0, ("b", (32,), 0, bytes(128))]))
    at = raw.find(b"b") + 1 + 4 + 8 + 4
    struct.pack_into("<Q", raw, at, 8)
    for name, data in {"misaligned": bytes(raw),
                       "duplicate": gguf_bytes([], [t0, t0]),
                       "dims5": gguf_bytes([], [("c", (32, 1, 1, 1, 1), 0, bytes(128))]),
                       "alignment": gguf_bytes([("general.alignment", U32, 48)], [t0], alignment=48)}.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        assert _rc_of_open(p) == nm.E_FORMAT, name


def test_not_an_expert_stack(tmp_path):
    path = tmp_path / "flat.gguf"
    write_gguf(path, [], [("blk.0.ffn_gate_exps.weight", (256, 8), O.Q4_K, bytes(8 * 144))])
    with GgufFile(path) as f:
        with pytest.raises(nm.NaiwaError) as ei:
            f.expert_stack(0, PROJ_GATE)
        assert ei.value.rc == nm.E_UNSUPPORTED
        with pytest.raises(nm.NaiwaError):
            f.expert_stack(0, PROJ_DOWN)  # missing
