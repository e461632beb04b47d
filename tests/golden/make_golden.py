"""Writes tests/golden/unet_f64.json: input/output vectors of the Diffusion Policy U-Net computed by
the independent float64 PyTorch restatement in tests/unet_ref.py (not by the oracle).

Inputs are the synthetic tiny checkpoint (flowedge_amd.checkpoint, seed 0) and the replica of the
reference's DiffusionFixture model (test/core_model_tests.cc:170-270); the file also records
each checkpoint's SHA-256 so a change of the generator is detected instead of silently changing
the vectors.  Run from the repository root:  python -m tests.golden.make_golden
"""

from __future__ import annotations

import hashlib
import json
import math
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from flowedge_amd import checkpoint as ck  # noqa: E402
from tests import unet_ref  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "unet_f64.json")


def sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def ddim_f64(tensors, cond, noise, steps: int, T: int, clip: float, amin, amax):
    """DDIM (diffusion.cc:979-1034) in float64 around the float64 U-Net."""
    ac = unet_ref.alphas_cumprod_f64(T)
    x = np.asarray(noise, np.float64).copy()
    ratio = T // steps
    for i in range(steps):
        ts = (steps - 1 - i) * ratio
        prev = ts - ratio
        at = ac[ts]
        ap = ac[prev] if prev >= 0 else 1.0
        e = unet_ref.torch_unet_eps(tensors, cond, x, float(ts))
        x0 = np.clip((x - math.sqrt(1 - at) * e) / math.sqrt(at), -clip, clip)
        x = math.sqrt(ap) * x0 + math.sqrt(1 - ap) * e
    return (x + 1) * 0.5 * (np.asarray(amax) - np.asarray(amin)) + np.asarray(amin)


def main():
    d = tempfile.mkdtemp()
    tiny = ck.cached_checkpoint("tiny", d)
    spec = ck.SPECS["tiny"]
    tt = ck.read_safetensors(tiny)
    cond, noise = ck.inputs(spec)
    golden = {"tiny": {"checkpoint_sha256": sha256(tiny), "cond_seed": 1, "noise_seed": 2,
                       "eps": {}, "ddim10": None}}
    for t in (99.0, 50.0, 0.3):
        golden["tiny"]["eps"][str(t)] = unet_ref.torch_unet_eps(tt, cond[0], noise[0], t).tolist()
    golden["tiny"]["ddim10"] = ddim_f64(tt, cond[0], noise[0], 10, spec.train_timesteps, 1.0,
                                        -1.0, 1.0).tolist()
    fx = unet_ref.write_fixture(os.path.join(d, "fixture.safetensors"))
    ft = ck.read_safetensors(fx)
    meta = [float(v) for v in ft["dp.meta"]]
    A, H, C = int(meta[1]), int(meta[2]), int(meta[5])
    fcond = unet_ref.seq(C, 0.17, 0.3)
    fsample = unet_ref.seq(H * A, 0.11, 0.7).reshape(H, A)
    golden["fixture"] = {"checkpoint_sha256": sha256(fx), "cond": fcond.tolist(),
                         "sample": fsample.tolist(), "t": 7.0,
                         "eps": unet_ref.torch_unet_eps(ft, fcond, fsample, 7.0).tolist()}
    with open(OUT, "w") as f:
        json.dump(golden, f, indent=1)
    print(OUT)


if __name__ == "__main__":
    main()
