"""The split final update against the one-workgroup update.

With a 512-channel final width in 8 GroupNorm groups and up to 16 samples, the final GroupNorm +
Mish + 1x1 conv + sampler update runs as one wavefront per (sample, group); the sample's last
wavefront to finish (an arrival counter it resets) adds the groups' partial outputs in group
order and applies the update.  It reduces in the same order as the one-workgroup kernel
(FLOWEDGE_SPLIT_UPDATE=0 at load), so the actions must agree bit for bit, and repeated ticks must
repeat exactly (a counter left non-zero would skip the next update).
"""

from __future__ import annotations

import numpy as np
import pytest

import flowedge_amd
from flowedge_amd import checkpoint as ck

pytestmark = pytest.mark.gpu


def say(msg: str):
    print(msg, flush=True)


def engines(path, monkeypatch):
    split = flowedge_amd.Engine(path)
    monkeypatch.setenv("FLOWEDGE_SPLIT_UPDATE", "0")
    whole = flowedge_amd.Engine(path)
    monkeypatch.delenv("FLOWEDGE_SPLIT_UPDATE")
    return split, whole


@pytest.mark.parametrize("work", ["pusht", "bimanual"])
def test_split_update_equals_one_workgroup(ckpt_dir, monkeypatch, work):
    spec = ck.SPECS[work]
    path = ck.cached_checkpoint(work, ckpt_dir)
    cond, noise = ck.inputs(spec, batch=3)
    split, whole = engines(path, monkeypatch)
    with split, whole:
        for scheduler, seed in (("ddim", 0), ("ddpm", 7)):
            say(f"{work} B=1 {scheduler}-10 split vs one-workgroup update")
            a = split.sample_diffusion(cond[0], noise[0], steps=10, scheduler=scheduler, seed=seed)
            b = whole.sample_diffusion(cond[0], noise[0], steps=10, scheduler=scheduler, seed=seed)
            assert np.all(np.isfinite(a))
            assert np.array_equal(a, b)
            again = split.sample_diffusion(cond[0], noise[0], steps=10, scheduler=scheduler,
                                           seed=seed)
            assert np.array_equal(a, again)
        say(f"{work} B=3 ddim-10 split vs one-workgroup update")
        a = split.sample_diffusion_batch(cond, noise, steps=10)
        b = whole.sample_diffusion_batch(cond, noise, steps=10)
        assert np.array_equal(a, b)
        assert np.array_equal(split.sample_diffusion_batch(cond, noise, steps=10), a)


@pytest.mark.parametrize("method,steps", [("euler", 10), ("rk4", 4)])
def test_split_update_flow(ckpt_dir, monkeypatch, method, steps):
    spec = ck.SPECS["flow"]
    path = ck.cached_checkpoint("flow", ckpt_dir)
    cond, x0 = ck.inputs(spec)
    split, whole = engines(path, monkeypatch)
    with split, whole:
        say(f"flow {method}-{steps} split vs one-workgroup update")
        a = np.empty((spec.horizon, spec.action_dim), np.float32)
        b = np.empty_like(a)
        split.sample_condition(cond[0], x0[0], a, steps=steps, method=method)
        whole.sample_condition(cond[0], x0[0], b, steps=steps, method=method)
        assert np.all(np.isfinite(a))
        assert np.array_equal(a, b)
