"""The persistent batch-1 tick against the per-layer graphs.

A persistent tick runs every convolution step of every U-Net evaluation in one launch of one
workgroup per CU, handing activations over through device-coherent memory; the per-layer path
replays a graph of one launch per convolution.  With input-channel slicing off
(FLOWEDGE_SLICES=1), the per-layer path runs the same convolution and update code on the same
plans as the tick kernel, so their actions must agree bit for bit; the per-layer path is itself
held to the oracle by test_gpu_parity.py.  Repeated ticks must be bit-identical (a stale read in
the hand-off would show up as run-to-run differences).  FLOWEDGE_PERSISTENT=1 at load selects
the persistent tick (which runs unsliced).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import flowedge_amd
import oracle
from flowedge_amd import checkpoint as ck
from tests import unet_ref

pytestmark = pytest.mark.gpu


def say(msg: str):
    print(msg, flush=True)


def engines(path, monkeypatch):
    monkeypatch.setenv("FLOWEDGE_PERSISTENT", "1")
    chain = flowedge_amd.Engine(path)
    monkeypatch.delenv("FLOWEDGE_PERSISTENT")
    monkeypatch.setenv("FLOWEDGE_SLICES", "1")
    layers = flowedge_amd.Engine(path)
    monkeypatch.delenv("FLOWEDGE_SLICES")
    say(f"persistent: {chain.persistent_tick} ({chain.persistent_tick_reason!r}); "
        f"reference engine: {layers.persistent_tick} ({layers.persistent_tick_reason!r})")
    assert chain.persistent_tick, chain.persistent_tick_reason
    assert not layers.persistent_tick
    return chain, layers


@pytest.mark.parametrize("steps,scheduler,seed", [(10, "ddim", 0), (1, "ddim", 0),
                                                  (100, "ddim", 0), (10, "ddpm", 42)])
def test_tiny_persistent_equals_layers(ckpt_dir, monkeypatch, steps, scheduler, seed):
    spec = ck.SPECS["tiny"]
    path = ck.cached_checkpoint("tiny", ckpt_dir)
    cond, noise = ck.inputs(spec)
    chain, layers = engines(path, monkeypatch)
    with chain, layers:
        say(f"tiny {scheduler}-{steps} persistent vs per-layer")
        a = chain.sample_diffusion(cond[0], noise[0], steps=steps, scheduler=scheduler, seed=seed)
        b = layers.sample_diffusion(cond[0], noise[0], steps=steps, scheduler=scheduler, seed=seed)
        assert np.array_equal(a, b)
        assert chain.persistent_tick


@pytest.mark.parametrize("method,steps", [("euler", 10), ("heun", 3), ("rk4", 4)])
def test_flow_small_persistent_equals_layers(ckpt_dir, monkeypatch, method, steps):
    spec = ck.UNetSpec(dims=(64, 128, 256), action_dim=7, cond_dim=32, prediction=1)
    path = unet_ref.write_variant(os.path.join(ckpt_dir, "flow_small_gpu.safetensors"), spec)
    cond, x0 = ck.inputs(spec)
    chain, layers = engines(path, monkeypatch)
    with chain, layers:
        say(f"flow small {method}-{steps} persistent vs per-layer")
        a = np.empty((spec.horizon, spec.action_dim), np.float32)
        b = np.empty_like(a)
        chain.sample_condition(cond[0], x0[0], a, steps=steps, method=method)
        layers.sample_condition(cond[0], x0[0], b, steps=steps, method=method)
        assert np.array_equal(a, b)


def test_pusht_persistent_equals_layers_and_repeats(ckpt_dir, monkeypatch):
    import torch

    spec = ck.SPECS["pusht"]
    path = ck.cached_checkpoint("pusht", ckpt_dir)
    cond, noise = ck.inputs(spec)
    chain, layers = engines(path, monkeypatch)
    with chain, layers:
        say("pusht DDIM-10 / DDPM-10 persistent vs per-layer")
        a = chain.sample_diffusion(cond[0], noise[0], steps=10)
        assert np.array_equal(a, layers.sample_diffusion(cond[0], noise[0], steps=10))
        d = chain.sample_diffusion(cond[0], noise[0], steps=10, scheduler="ddpm", seed=5)
        assert np.array_equal(d, layers.sample_diffusion(cond[0], noise[0], steps=10,
                                                         scheduler="ddpm", seed=5))
        # Device-resident ticks (the benchmark's call), repeated: bit-identical every time.
        dev = torch.device("cuda:0")
        dc, dn = torch.from_numpy(cond).to(dev), torch.from_numpy(noise).to(dev)
        out = torch.empty((1, spec.horizon, spec.action_dim), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        say("pusht DDIM-10 x 50 device-resident persistent ticks")
        for i in range(50):
            chain.sample_device(0, dc.data_ptr(), dn.data_ptr(), 1, 10, 0, 0, out.data_ptr())
            assert np.array_equal(out.cpu().numpy()[0], a), f"tick {i} differs"
        say(f"pusht persistent tick device time {chain.last_device_ms:.3f} ms")
        assert chain.persistent_tick
        # Other calls between ticks (eager denoise, matrix-core batch) leave it consistent.
        chain.diffusion_denoise(cond[0], noise[0], 30.0)
        cb, nb = ck.inputs(spec, batch=6)
        chain.sample_diffusion_batch(cb, nb, steps=2)
        assert np.array_equal(chain.sample_diffusion(cond[0], noise[0], steps=10), a)


def test_flow_full_persistent_matches_oracle(ckpt_dir, monkeypatch):
    spec = ck.SPECS["flow"]
    path = ck.cached_checkpoint("flow", ckpt_dir)
    cond, x0 = ck.inputs(spec)
    o = oracle.Oracle(path, threads=8)
    monkeypatch.setenv("FLOWEDGE_PERSISTENT", "1")
    with flowedge_amd.Engine(path) as e:
        assert e.persistent_tick, e.persistent_tick_reason
        for method, steps in (("rk4", 4), ("euler", 10)):
            out = np.empty((spec.horizon, spec.action_dim), np.float32)
            e.sample_condition(cond[0], x0[0], out, steps=steps, method=method)
            err = float(np.max(np.abs(out.astype(np.float64) -
                                      o.sample_flow(cond[0], x0[0], steps,
                                                    flowedge_amd.SOLVERS[method]))))
            say(f"flow {method}-{steps} persistent max err {err:.3e}")
            assert err <= 1e-4


def test_long_solve_uses_per_layer_graph(ckpt_dir, monkeypatch):
    # More evaluations than a persistent tick's table holds (flow RK4-40 = 160): per-layer graphs,
    # same values as a persistent-free engine would give (held to the oracle).
    spec = ck.UNetSpec(dims=(64, 128, 256), action_dim=7, cond_dim=32, prediction=1)
    path = unet_ref.write_variant(os.path.join(ckpt_dir, "flow_small_gpu.safetensors"), spec)
    cond, x0 = ck.inputs(spec)
    o = oracle.Oracle(path)
    monkeypatch.setenv("FLOWEDGE_PERSISTENT", "1")
    with flowedge_amd.Engine(path) as e:
        out = np.empty((spec.horizon, spec.action_dim), np.float32)
        e.sample_condition(cond[0], x0[0], out, steps=40, method="rk4")
        err = float(np.max(np.abs(out - o.sample_flow(cond[0], x0[0], 40, 2))))
        assert err <= 1e-4
        assert e.persistent_tick
