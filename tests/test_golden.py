"""Committed golden vectors (tests/golden/unet_f64.json, written by tests/golden/make_golden.py from
the independent float64 PyTorch U-Net, not from the oracle): the oracle on the CPU and the HIP
path through the C ABI are both held to them.

Tolerances: oracle epsilon 2e-5 (tiny) / 2e-6 (fixture) absolute, DDIM-10 actions 1e-4; HIP
path 1e-4 throughout (fp32 contract bound, action scale 1).
"""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from flowedge_amd import checkpoint as ck
from tests import unet_ref

GOLDEN = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                     "unet_f64.json")))


def sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


@pytest.fixture(scope="module")
def tiny(ckpt_dir):
    return ck.cached_checkpoint("tiny", ckpt_dir)


@pytest.fixture(scope="module")
def fixture_model(ckpt_dir):
    return unet_ref.write_fixture(os.path.join(ckpt_dir, "golden_fixture.safetensors"))


def test_golden_checkpoints_unchanged(tiny, fixture_model):
    assert sha256(tiny) == GOLDEN["tiny"]["checkpoint_sha256"]
    assert sha256(fixture_model) == GOLDEN["fixture"]["checkpoint_sha256"]


def test_oracle_matches_golden_tiny(tiny):
    o = oracle.Oracle(tiny)
    cond, noise = ck.inputs(ck.SPECS["tiny"])
    for t, want in GOLDEN["tiny"]["eps"].items():
        np.testing.assert_allclose(o.denoise(cond[0], noise[0], float(t)), want, atol=2e-5, rtol=0)
    np.testing.assert_allclose(o.sample(cond[0], noise[0], 10), GOLDEN["tiny"]["ddim10"],
                               atol=1e-4, rtol=0)


def test_oracle_matches_golden_fixture(fixture_model):
    g = GOLDEN["fixture"]
    o = oracle.Oracle(fixture_model)
    got = o.denoise(np.array(g["cond"], np.float32), np.array(g["sample"], np.float32), g["t"])
    np.testing.assert_allclose(got, g["eps"], atol=2e-6, rtol=0)


@pytest.mark.gpu
def test_hip_matches_golden(tiny, fixture_model):
    import flowedge_amd

    cond, noise = ck.inputs(ck.SPECS["tiny"])
    with flowedge_amd.Engine(tiny) as e:
        for t, want in GOLDEN["tiny"]["eps"].items():
            got = e.diffusion_denoise(cond[0], noise[0], float(t))
            assert float(np.max(np.abs(got - np.array(want)))) <= 1e-4
        got = e.sample_diffusion(cond[0], noise[0], steps=10)
        assert float(np.max(np.abs(got - np.array(GOLDEN["tiny"]["ddim10"])))) <= 1e-4
    g = GOLDEN["fixture"]
    with flowedge_amd.Engine(fixture_model) as e:
        got = e.diffusion_denoise(np.array(g["cond"], np.float32),
                                  np.array(g["sample"], np.float32), g["t"])
        assert float(np.max(np.abs(got - np.array(g["eps"])))) <= 1e-4
