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
