"""Build recipe for the gfx950 library (``libflowedge_amd.so``), in-tree.

One hipcc invocation compiles the host runtime (C ABI, loader, graph cache) and the device
kernels for ``--offload-arch=gfx950``.  Packed-FP32 instructions are disabled for all device code.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libflowedge_amd.so")
SOURCES = ["csrc/engine.cpp", "csrc/safetensors.cpp", "csrc/kernels.hip", "csrc/conv_fused.hip",
           "csrc/conv_same5.hip", "csrc/conv_same3.hip", "csrc/conv_resample.hip",
           "csrc/conv_mfma.hip", "csrc/conv_mfma_bf16.hip", "csrc/conv_general.hip",
           "csrc/identity.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def command(out: str = LIB) -> list[str]:
    return [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", os.path.join(ROOT, "include"),
            *[os.path.join(HERE, s) for s in SOURCES], "-o", out]


def build(verbose: bool = False) -> str:
    tmp = LIB + f".tmp{os.getpid()}"
    res = subprocess.run(command(tmp), capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libflowedge_amd.so")
    if verbose:
        sys.stderr.write(res.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
