"""Build recipe for the gfx950 library (``libflowedge_amd.so``), in-tree.

Each translation unit (host runtime, loader, device kernels) is compiled by its own hipcc process
for ``--offload-arch=gfx950`` into ``flowedge_amd/_build/``, in parallel, and the objects are
linked into one shared library.  Packed-FP32 instructions are disabled for all device code.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libflowedge_amd.so")
OBJDIR = os.path.join(HERE, "_build")
SOURCES = ["csrc/engine.cpp", "csrc/safetensors.cpp", "csrc/kernels.hip", "csrc/conv_fused.hip",
           "csrc/conv_same5.hip", "csrc/conv_same3.hip", "csrc/conv_resample.hip",
           "csrc/conv_slice.hip", "csrc/conv_slice_s16.hip", "csrc/conv_slice_l16.hip",
           "csrc/conv_slice_s32.hip", "csrc/conv_slice_l32.hip", "csrc/conv_slice_s64.hip",
           "csrc/conv_slice_l64.hip",
           "csrc/conv_mfma.hip", "csrc/conv_mfma_bf16.hip", "csrc/conv_general.hip",
           "csrc/identity.cpp", "csrc/scratch.hip", "csrc/chain.hip", "csrc/encoder.hip",
           "csrc/encoder.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=on: a multiply and an add fuse only within one expression, so a kernel body
# rounds the same way in every kernel it is inlined into (the persistent tick kernel and the
# per-layer kernels give bit-identical results); "fast" would also fuse across statements
# wherever the surrounding code places both in one basic block.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=on",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(ROOT, "include")]


def _obj(src: str) -> str:
    return os.path.join(OBJDIR, os.path.basename(src) + ".o")


def compile_command(src: str, obj: str) -> list[str]:
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    return [HIPCC, *FLAGS, "-c", *lang, os.path.join(HERE, src), "-o", obj]


def link_command(out: str) -> list[str]:
    return [HIPCC, "--offload-arch=gfx950", "-fPIC", "-shared", "--hip-link",
            *[_obj(s) for s in SOURCES], "-o", out]


def build(verbose: bool = False, jobs: int | None = None) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 1)))

    def run(cmd):
        return subprocess.run(cmd, capture_output=True, text=True)

    with ThreadPoolExecutor(jobs) as pool:
        results = list(pool.map(lambda s: (s, run(compile_command(s, _obj(s)))), SOURCES))
    failed = [(s, r) for s, r in results if r.returncode != 0]
    for s, r in results:
        if verbose or r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
    if failed:
        raise RuntimeError("hipcc failed on " + ", ".join(s for s, _ in failed))
    tmp = LIB + f".tmp{os.getpid()}"
    res = run(link_command(tmp))
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("linking libflowedge_amd.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
