"""Properties of the generated gfx950 code that the fused decode kernel relies on
(CPU only: hipcc cross-compiles csrc/stack_fused.hip to assembly).

The kernel issues its global -> LDS DMA as inline assembly that sets M0 and then
runs global_load_lds_dwordx4, so that the compiler's wait tracking does not make
every later LDS read wait for every DMA in flight.  M0 is a reserved register
and the compiler does not honour a clobber of it; the code is sound only while
M0 is written by those sequences alone and read by nothing else."""
import importlib.util
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "naiwa-rs_amd")


def _build_module():
    spec = importlib.util.spec_from_file_location("naiwa_build", os.path.join(PKG, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def fused_asm(tmp_path_factory):
    b = _build_module()
    if not os.path.exists(b.HIPCC):
        pytest.skip("hipcc is not installed")
    out = tmp_path_factory.mktemp("asm") / "stack_fused.s"
    flags = [f for f in b.CFLAGS if f != "-fPIC"]
    cmd = [b.HIPCC, *flags, "-I", b.CSRC, "--cuda-device-only", "-S",
           os.path.join(b.CSRC, "stack_fused.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stderr[-2000:]
    # instructions only: comments and directives dropped
    lines = [l.split(";")[0].strip() for l in out.read_text().splitlines()]
    return [l for l in lines if l and not l.startswith(".")]


def test_m0_is_written_only_to_address_an_lds_dma(fused_asm):
    uses = [i for i, l in enumerate(fused_asm) if re.search(r"\bm0\b", l)]
    assert uses, "no LDS DMA found: the kernel's gate/up staging changed"
    for i in uses:
        assert fused_asm[i].startswith("s_mov_b32 m0, s"), fused_asm[i]
        assert fused_asm[i + 1] == "s_nop 0", fused_asm[i + 1]
        assert fused_asm[i + 2].startswith("global_load_lds_dwordx4 "), fused_asm[i + 2]
    dmas = [l for l in fused_asm if l.startswith("global_load_lds")]
    assert len(dmas) == len(uses)


def test_no_instruction_reads_m0_implicitly(fused_asm):
    implicit = re.compile(r"^(s_movrel|v_movrel|s_set_gpr_idx|s_sendmsg|ds_gws|v_interp|s_ttracedata|"
                          r"buffer_load\S*\s.*\blds\b|ds_append|ds_consume)")
    hits = [l for l in fused_asm if implicit.match(l)]
    assert not hits, hits[:5]


def _kernel_vgprs(src: str, tmp_path) -> dict:
    """VGPRs of every kernel in csrc/<src>, from the code object metadata of its gfx950
    assembly, by mangled name."""
    b = _build_module()
    if not os.path.exists(b.HIPCC):
        pytest.skip("hipcc is not installed")
    out = tmp_path / (src + ".s")
    flags = [f for f in b.CFLAGS if f != "-fPIC"]
    r = subprocess.run([b.HIPCC, *flags, "-I", b.CSRC, "--cuda-device-only", "-S", os.path.join(b.CSRC, src),
                        "-o", str(out)], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stderr[-2000:]
    text = out.read_text()
    meta = text[text.index("amdhsa.kernels"):]
    vgprs = {}
    for entry in meta.split("\n  - ")[1:]:
        name = re.search(r"\.name:\s+(\S+)", entry)
        count = re.search(r"\.vgpr_count:\s+(\d+)", entry)
        if name and count:
            vgprs[name.group(1)] = int(count.group(1))
    return vgprs


def test_staged_gate_up_leaves_registers_for_the_copy_kernel(tmp_path):
    """Staged gate/up blocks of small calls wait for the upload flag while the copy kernel
    on the other stream has still to run, so however many of them a SIMD holds, the copy
    kernel's wave must still fit beside them (512 VGPRs a SIMD lane, allocated 8 at a
    time; the LDS can only lower the count).  A build where they filled every register
    made every wait run out."""
    gate_up = {n: v for n, v in _kernel_vgprs("decode.hip", tmp_path).items() if "gate_up_staged_kernel" in n}
    copies = {n: v for n, v in _kernel_vgprs("upload.hip", tmp_path).items() if "copy_batch_kernel" in n}
    assert gate_up and copies
    alloc = lambda v: (v + 7) // 8 * 8
    copy_need = max(alloc(v) for v in copies.values())
    for name, v in gate_up.items():
        waves = min(8, 512 // alloc(v))
        assert waves * alloc(v) + copy_need <= 512, (name, v, waves, copy_need)
