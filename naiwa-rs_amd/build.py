"""Build libnaiwa_moe.so (gfx950) in-tree with hipcc.

Every .hip/.cpp file under csrc/ is compiled to an object with
--offload-arch=gfx950 and linked into naiwa-rs_amd/libnaiwa_moe.so, which the
ctypes binding in naiwa_moe/ loads.  Packed-FP32 instruction selection is
switched off for device code.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libnaiwa_moe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("NAIWA_OFFLOAD_ARCH", "gfx950")

CFLAGS = [
    "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


# Host-code sanitizers (CPU runs only): every -fsanitize flag applies to the host
# compilation alone (-Xarch_host before it); device code is built as usual.
SANITIZE = {
    "address": ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"],
    "thread": ["-Xarch_host", "-fsanitize=thread"],
}


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src: str, build_dir: str = BUILD, extra: tuple = ()) -> str:
    obj = os.path.join(build_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, *extra, "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    noise = "is not a recognized feature for this target"
    rest = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if rest.strip():
        sys.stderr.write(rest + "\n")
    return obj


def build(jobs: int = 8, sanitize: str | None = None) -> str:
    """Build the library; with sanitize ("address" or "thread") an instrumented copy of
    the host code goes to naiwa-rs_amd/_san/libnaiwa_moe_<sanitize>.so instead (for CPU
    test runs with the matching runtime preloaded; never for the GPU)."""
    extra = tuple(SANITIZE[sanitize]) if sanitize else ()
    build_dir = BUILD if not sanitize else os.path.join(HERE, "_san", "obj_" + sanitize)
    lib = LIB if not sanitize else os.path.join(HERE, "_san", f"libnaiwa_moe_{sanitize}.so")
    os.makedirs(build_dir, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s_: _compile(s_, build_dir, extra), srcs))
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *extra, "-o", tmp, *objs,
           "-Wl,-rpath,/opt/rocm/lib", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser()
    ap.add_argument("--sanitize", choices=sorted(SANITIZE), default=None)
    print(build(sanitize=ap.parse_args().sanitize))
