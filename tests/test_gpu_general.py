"""GPU parity of the general-shape kernels against the CPU oracle.

The checkpoints here have shapes the specialised kernels have no instance for: kernel sizes 1
and 7, horizons 6 / 12 / 64, 64 GroupNorm groups, widths that are not multiples of 16, width *
length above 8192, 70 action dims and a final width of 1088 (tests/unet_ref.py GENERAL_SPECS).
Each is valid for the reference (diffusion.cc:391-427), so the engine must load and sample it.
Tolerance as the other fp32 parity tests: max |err| <= 1e-4 in action units; BF16 weights are
held to the same bound because the oracle runs on the identical BF16-rounded values.
"""

from __future__ import annotations

import dataclasses
import os

import numpy as np
import pytest

import flowedge_amd
import oracle
from flowedge_amd import checkpoint as ck
from tests import unet_ref

pytestmark = pytest.mark.gpu

TOL = 1e-4


def say(msg: str):
    print(msg, flush=True)


def maxerr(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


@pytest.fixture(scope="module", params=sorted(unet_ref.GENERAL_SPECS))
def general(request, ckpt_dir):
    name = request.param
    spec = unet_ref.GENERAL_SPECS[name]
    path = unet_ref.write_variant(os.path.join(ckpt_dir, f"general_{name}.safetensors"), spec)
    return name, spec, path, oracle.Oracle(path)


def test_general_shapes_batch1(general):
    name, spec, path, o = general
    cond, noise = ck.inputs(spec)
    with flowedge_amd.Engine(path) as e:
        paths = e.conv_paths(1)
        say(f"{name} batch 1: {paths.count('general')} of {len(paths)} convolutions general")
        # Kernel 7, lengths 6 / 12 / 3 and width * length 16384 have no specialised instance.
        # The others reach the general kernels outside the convolutions: g64_k3 in the GroupNorm
        # prologue (64 groups; its normalised convolutions then run on the matrix cores even at
        # batch 1), a70 (70 action dims) and k1_c1088 (final width 1088) in the final update.
        if name in ("k7_h6_g3", "h12_stages3", "h64_wide"):
            assert "general" in paths
        elif name == "g64_k3":
            assert "matrix" in paths
        got = e.diffusion_denoise(cond[0], noise[0], 17.0)
        assert maxerr(got, o.denoise(cond[0], noise[0], 17.0)) <= TOL
        got = e.sample_diffusion(cond[0], noise[0], steps=5)
        assert maxerr(got, o.sample(cond[0], noise[0], 5, 0, 0)) <= TOL
        got = e.sample_diffusion(cond[0], noise[0], steps=5, scheduler="ddpm", seed=3)
        assert maxerr(got, o.sample(cond[0], noise[0], 5, 1, 3)) <= TOL


def test_general_shapes_batched(general):
    name, spec, path, o = general
    B = 5  # above the matrix-core threshold
    cond, noise = ck.inputs(spec, batch=B)
    with flowedge_amd.Engine(path) as e:
        paths = e.conv_paths(B)
        say(f"{name} batch {B}: " + ", ".join(f"{p} {paths.count(p)}" for p in sorted(set(paths))))
        got = e.sample_diffusion_batch(cond, noise, steps=5)
        want = o.sample_batch(cond, noise, 5, workers=8)
        assert maxerr(got, want) <= TOL
        eps = e.diffusion_denoise_batch(cond, noise, 33.0)
        for b in (0, B - 1):
            assert maxerr(eps[b], o.denoise(cond[b], noise[b], 33.0)) <= TOL


@pytest.mark.parametrize("method,steps", [("rk4", 3), ("heun", 4)])
def test_general_shape_flow(ckpt_dir, method, steps):
    spec = dataclasses.replace(unet_ref.GENERAL_SPECS["h12_stages3"], prediction=1)
    path = unet_ref.write_variant(os.path.join(ckpt_dir, "general_flow_h12.safetensors"), spec)
    o = oracle.Oracle(path)
    B = 5
    cond, x0 = ck.inputs(spec, batch=B)
    say(f"general flow h12 {method} steps={steps}")
    with flowedge_amd.Engine(path) as e:
        out = np.empty((spec.horizon, spec.action_dim), np.float32)
        e.sample_condition(cond[0], x0[0], out, steps=steps, method=method)
        m = flowedge_amd.SOLVERS[method]
        assert maxerr(out, o.sample_flow(cond[0], x0[0], steps, m)) <= TOL
        got = e.sample_condition_batch(cond, x0, steps=steps, method=method)
        assert maxerr(got, o.sample_batch(cond, x0, steps, 1, m, workers=8)) <= TOL


def test_general_shape_bf16_weights(ckpt_dir):
    spec = dataclasses.replace(unet_ref.GENERAL_SPECS["k7_h6_g3"], bf16_weights=True)
    path = unet_ref.write_variant(os.path.join(ckpt_dir, "general_k7_bf16.safetensors"), spec)
    o = oracle.Oracle(path)
    B = 9  # above the BF16 matrix-core threshold (5)
    cond, noise = ck.inputs(spec, batch=B)
    say("general k7 h6 BF16 weights, batch 1 and 9")
    with flowedge_amd.Engine(path) as e:
        assert e.model_metadata["precision"] in (2, 3)
        got = e.sample_diffusion(cond[0], noise[0], steps=5)
        assert maxerr(got, o.sample(cond[0], noise[0], 5, 0, 0)) <= TOL
        got = e.sample_diffusion_batch(cond, noise, steps=5)
        assert maxerr(got, o.sample_batch(cond, noise, 5, workers=8)) <= TOL
