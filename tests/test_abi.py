"""The C-ABI library loads without a GPU and exports every symbol the header declares."""
import ctypes
import os
import re

import naiwa_moe
from naiwa_moe import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in sorted(os.listdir(os.path.join(ROOT, "include")))
           if f.endswith(".h")]


def declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?([A-Za-z_][\w]*)\s*\*?\s*\b([a-z_][a-z0-9_]*)\s*\(",
                             text, flags=re.M):
            if m.group(1) != "typedef":   # function-pointer typedefs declare no symbol
                names.append(m.group(2))
    return sorted(set(names))


def test_header_declares_the_reference_doorbell_ffi():
    names = declared_functions()
    for n in ("doorbell_alloc_mapped", "doorbell_free_host", "doorbell_get_device_ptr",
              "doorbell_ring", "doorbell_copy_f32", "doorbell_wait_copy_f32"):
        assert n in names


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_declares_every_header_symbol():
    assert set(declared_functions()) <= set(_lib.SIGNATURES)


def test_library_loads_without_a_device():
    L = naiwa_moe.lib()
    assert L.naiwa_status_string(-3) == b"wait timed out"
    assert L.naiwa_projection_bytes(naiwa_moe.Q4_K, 768, 2048) == 884736
    assert L.naiwa_projection_bytes(naiwa_moe.Q8_0, 2048, 1024) == 2048 * 32 * 34
    assert L.naiwa_projection_bytes(naiwa_moe.Q4_K, 2048, 1408) == -1


def test_argument_errors_need_no_device():
    L = naiwa_moe.lib()
    # invalid shapes are rejected before anything is launched
    assert L.naiwa_moe_gather(None, -1, 4, None, None, None, 0) == naiwa_moe._lib.E_INVALID
    assert L.naiwa_router_topk(None, naiwa_moe.BF16, None, 1, 12, 8, 2, 0, None, None, None, 0) \
        == naiwa_moe._lib.E_INVALID
    assert L.naiwa_router_topk(None, 99, None, 1, 16, 8, 2, 0, None, None, None, 0) \
        == naiwa_moe._lib.E_UNSUPPORTED


def _fake_bank(n, k, dtype, slots=8):
    """A bank descriptor whose base is a made-up (aligned, never dereferenced) address."""
    stride = (naiwa_moe.lib().naiwa_projection_bytes(dtype, n, k) + 255) & ~255
    return _lib.Bank(0x7f0000000000, stride, slots, n, k, dtype)


def test_noalloc_capacity_is_checked_before_any_device_call():
    """naiwa_moe_decode_noalloc refuses a call one pair past its fixed array with
    NAIWA_E_TOO_LARGE before it touches a device (none here: the made-up
    pointers would fault if anything ran), and the size query names the limit:
    56 pairs (28 rows of top-2) at H 4096 / I 14336 in Q4_K, 339 rows of top-8 at
    H 2048 / I 768."""
    L = naiwa_moe.lib()
    cap = 8 << 20   # NAIWA_DECODE_NOALLOC_SCRATCH_BYTES
    Q4K = naiwa_moe.Q4_K
    fake = ctypes.c_void_p(0x7f0000100000)
    for H, I, width, rows_max in ((4096, 14336, 2, 28), (2048, 768, 8, 339), (4096, 14336, 1, 55)):
        assert 0 < L.naiwa_moe_decode_scratch_bytes(rows_max, width, H, I, Q4K) <= cap
        assert L.naiwa_moe_decode_scratch_bytes(rows_max + 1, width, H, I, Q4K) > cap
        g, u, d = _fake_bank(I, H, Q4K), _fake_bank(I, H, Q4K), _fake_bank(H, I, Q4K)
        rc = L.naiwa_moe_decode_noalloc(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), fake, naiwa_moe.BF16,
                                        fake, fake, rows_max + 1, width, naiwa_moe.ACT_SILU, fake, 0, 0)
        assert rc == _lib.E_TOO_LARGE, (H, I, width, rc)
    # the staged-h path (<= 512 pairs, <= 16 per row) carries K-part dots and
    # costs more per pair than f32 h, so the limit is not monotone in the pairs
    fits = [r for r in range(1, 260) if L.naiwa_moe_decode_scratch_bytes(r, 6, 5120, 1536, Q4K) <= cap]
    assert fits == list(range(1, 56)) + list(range(86, 228))
    # the K-part dots: one f32 per K part, pair and hidden feature, on top of h
    s1 = L.naiwa_moe_decode_scratch_bytes(1, 1, 4096, 14336, Q4K)
    s2 = L.naiwa_moe_decode_scratch_bytes(1, 2, 4096, 14336, Q4K)
    assert s2 - s1 >= 7 * 4096 * 4
    assert L.naiwa_moe_decode_scratch_bytes(0, 8, 2048, 768, Q4K) == 0
    assert L.naiwa_moe_decode_scratch_bytes(1, 8, 2048, 770, Q4K) == -1
    assert L.naiwa_moe_decode_scratch_bytes(1, 8, 2048, 768, 99) == -1
