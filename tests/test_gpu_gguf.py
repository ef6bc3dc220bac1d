"""GPU: a MoE layer read from a GGUF checkpoint (tests/gguf_writer.py) -- the
router from blk.0.ffn_gate_inp.weight, every expert copied from the mapped
stacks into pinned host stacks and uploaded into slot banks in a shuffled slot
order -- routes and decodes like the oracle on the arrays the file was written
from: top-k bit-exact, outputs within the 1e-2 bar."""
import numpy as np
import pytest

import oracle as O
import synthetic as S
from gguf_writer import STRING, U32, expert_tensors, write_gguf

pytestmark = pytest.mark.gpu
TOL = 1e-2


def test_layer_from_gguf_decodes_like_the_oracle(gpu, tmp_path):
    nm = gpu
    from naiwa_moe.gguf import GgufFile

    H, I, E, k, rows = 1024, 512, 8, 2, 3
    dt = (O.Q4_K, O.Q4_K, O.Q8_0)
    g, u, d, r = S.layer(700, E, H, I, dt)
    path = tmp_path / "layer.gguf"
    write_gguf(path, [("general.architecture", STRING, "qwen3moe"), ("qwen3moe.expert_count", U32, E)],
               expert_tensors(0, g, u, d, r, H, I, dt))
    slot_of = np.array([5, 2, 7, 0, 3, 6, 1, 4], dtype=np.int32)
    with GgufFile(path) as f:
        assert f.meta_u64("qwen3moe.expert_count") == E
        stacks = f.host_stacks(0)
        router = f.tensor_bytes("blk.0.ffn_gate_inp.weight").view(np.float32).reshape(E, H).copy()
    banks = nm.LayerBanks(E, H, I, dt)
    copy = nm.Stream()
    print(f"[gguf] uploading {E} experts", flush=True)
    for e in range(E):
        nm.upload_expert(banks, int(slot_of[e]), stacks, e, copy.handle)
    copy.sync()

    x = S.activations_bf16(701, rows, H)
    xd = nm.DeviceBuffer.from_array(x)
    rd = nm.DeviceBuffer.from_array(router)
    ids_d, w_d = nm.DeviceBuffer(rows * k * 4), nm.DeviceBuffer(rows * k * 4)
    nm.router_topk(xd, nm.BF16, rd, rows, H, E, k, ids_d, w_d)
    nm.synchronize()
    ids = ids_d.download(np.uint32).reshape(rows, k)
    w = w_d.download(np.float32).reshape(rows, k)
    want_ids, want_w = O.topk(O.router_logits(O.from_bf16(x), r), k)
    assert np.array_equal(ids, want_ids)
    assert np.allclose(w, want_w, rtol=1e-5, atol=1e-7)

    slots = nm.DeviceBuffer.from_array(slot_of[ids].astype(np.uint32))
    out = nm.DeviceBuffer(rows * H * 4)
    print("[gguf] decode", flush=True)
    nm.indexed_moe_fused_decode(banks, xd, nm.BF16, slots, w_d, rows, k, out)
    nm.synchronize()
    got = out.download(np.float32).reshape(rows, H)
    gs, us, ds = O.stack(g, dt[0], I, H), O.stack(u, dt[1], I, H), O.stack(d, dt[2], H, I)
    want = O.fused_moe_decode(gs, us, ds, O.from_bf16(x), want_ids, want_w)
    err = S.max_rel_err(got, want)
    print(f"[gguf] max_rel_err={err:.3e}", flush=True)
    assert err < TOL
