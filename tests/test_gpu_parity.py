"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on identical inputs.

Tolerances (written per test): fp32 checkpoints must match within max |err| <= 1e-4 in action
units (action scale (max - min)/2 = 1 for the synthetic range [-1, 1]); BF16-weight checkpoints
are held to the same 1e-4 here because the oracle runs on the identical BF16-rounded values
(the contract bound for BF16 variants is 2e-2).  Batches below the matrix-core threshold
(FLOWEDGE_MFMA_BATCH, default 4 for F32 weights and 5 for BF16) run the batch-1 kernels and must
equal independent batch-1 calls bit for bit; larger batches run implicit GEMMs on the matrix
cores (another summation order) and are held to the oracle per sample at the same 1e-4.
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

TOL = 1e-4


def say(msg: str):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def tiny(ckpt_dir):
    return ck.cached_checkpoint("tiny", ckpt_dir)


@pytest.fixture(scope="module")
def tiny_engine(tiny):
    with flowedge_amd.Engine(tiny) as e:
        yield e


@pytest.fixture(scope="module")
def tiny_oracle(tiny):
    return oracle.Oracle(tiny)


def maxerr(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


@pytest.mark.parametrize("t", [99.0, 90.0, 50.0, 0.0, 0.3])
def test_tiny_denoise(tiny_engine, tiny_oracle, t):
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    say(f"tiny denoise t={t}")
    got = tiny_engine.diffusion_denoise(cond[0], noise[0], t)
    want = tiny_oracle.denoise(cond[0], noise[0], t)
    assert maxerr(got, want) <= 2e-5


@pytest.mark.parametrize("steps", [1, 3, 10, 100])
def test_tiny_ddim(tiny_engine, tiny_oracle, steps):
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    say(f"tiny DDIM steps={steps}")
    got = tiny_engine.sample_diffusion(cond[0], noise[0], steps=steps)
    want = tiny_oracle.sample(cond[0], noise[0], steps)
    assert maxerr(got, want) <= TOL
    assert np.all(got >= -1.0) and np.all(got <= 1.0)


@pytest.mark.parametrize("seed", [0, 42])
def test_tiny_ddpm(tiny_engine, tiny_oracle, seed):
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    say(f"tiny DDPM seed={seed}")
    got = tiny_engine.sample_diffusion(cond[0], noise[0], steps=10, scheduler="ddpm", seed=seed)
    want = tiny_oracle.sample(cond[0], noise[0], 10, 1, seed)
    assert maxerr(got, want) <= TOL
    again = tiny_engine.sample_diffusion(cond[0], noise[0], steps=10, scheduler="ddpm", seed=seed)
    assert np.array_equal(got, again)


def test_tiny_ddim_seed_independent_and_repeatable(tiny_engine):
    cond, noise = ck.inputs(ck.SPECS["tiny"])
    a = tiny_engine.sample_diffusion(cond[0], noise[0], steps=10, seed=1)
    b = tiny_engine.sample_diffusion(cond[0], noise[0], steps=10, seed=999)
    assert np.array_equal(a, b)


def test_tiny_batch_equals_independent_calls(tiny_engine):
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec, batch=3)  # below the matrix-core threshold: bit-exact
    say("tiny DDIM batch=3")
    batch = tiny_engine.sample_diffusion_batch(cond, noise, steps=10)
    for b in range(3):
        single = tiny_engine.sample_diffusion(cond[b], noise[b], steps=10)
        assert np.array_equal(batch[b], single)
    eps = tiny_engine.diffusion_denoise_batch(cond, noise, 50.0)
    for b in range(3):
        assert np.array_equal(eps[b], tiny_engine.diffusion_denoise(cond[b], noise[b], 50.0))


def test_no_device_allocation_after_load(tiny_engine):
    # core_model_tests.cc:475-495: device allocations do not change across sampling calls.
    cond, noise = ck.inputs(ck.SPECS["tiny"], batch=3)
    before = flowedge_amd.device_alloc_count()
    assert before >= 1
    tiny_engine.diffusion_denoise(cond[0], noise[0], 7.0)
    tiny_engine.sample_diffusion(cond[0], noise[0], steps=5)
    tiny_engine.sample_diffusion(cond[0], noise[0], steps=5, scheduler="ddpm", seed=42)
    tiny_engine.sample_diffusion_batch(cond, noise, steps=5)
    assert flowedge_amd.device_alloc_count() == before


def test_no_allocation_or_capture_after_first_call(tiny):
    # After the first call of a shape (or fe_engine_prepare) its sampling calls capture no graph
    # and leave the device's free memory unchanged (nothing allocated by the library or by the
    # HIP runtime on its behalf).
    import torch

    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec, batch=6)
    with flowedge_amd.Engine(tiny) as e:
        e.prepare(0, 6, 10, 0)
        e.sample_diffusion(cond[0], noise[0], steps=10)
        e.sample_diffusion(cond[0], noise[0], steps=10, scheduler="ddpm", seed=3)
        e.sample_diffusion_batch(cond, noise, steps=10)
        e.diffusion_denoise(cond[0], noise[0], 7.0)
        captures = e.graph_captures
        assert captures == 3
        allocs = flowedge_amd.device_alloc_count()
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(3):
            e.sample_diffusion(cond[0], noise[0], steps=10)
            e.sample_diffusion(cond[0], noise[0], steps=10, scheduler="ddpm", seed=3)
            e.sample_diffusion_batch(cond, noise, steps=10)
            e.diffusion_denoise(cond[0], noise[0], 7.0)
        assert e.graph_captures == captures
        assert flowedge_amd.device_alloc_count() == allocs
        assert torch.cuda.mem_get_info()[0] == free0


def test_diagnostics_then_first_sample(tiny, tiny_oracle):
    # Convolution diagnostics (listing and timing) before the first sampling graph of a fresh
    # engine: the graph is captured afterwards and matches the oracle.
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    with flowedge_amd.Engine(tiny) as e:
        convs = e.convolutions()
        assert len(convs) == 29
        assert e.time_convolutions([c["index"] for c in convs], batch=1, iters=2) > 0
        assert e.graph_captures == 0
        got = e.sample_diffusion(cond[0], noise[0], steps=10)
        assert e.graph_captures == 1
    assert maxerr(got, tiny_oracle.sample(cond[0], noise[0], 10)) <= TOL


def test_denoise_rejects_velocity_model(ckpt_dir):
    # engine_runtime.cc:476-479: no Diffusion Policy (epsilon) head -> status 4.
    spec = ck.UNetSpec(dims=(64, 128, 256), action_dim=7, cond_dim=32, prediction=1)
    path = unet_ref.write_variant(os.path.join(ckpt_dir, "flow_small_gpu.safetensors"), spec)
    cond, x = ck.inputs(spec)
    with flowedge_amd.Engine(path) as e:
        lib = flowedge_amd.lib()
        p = flowedge_amd._p
        c, n = np.ascontiguousarray(cond[0]), np.ascontiguousarray(x[0])
        out = np.empty((spec.horizon, spec.action_dim), np.float32)
        assert lib.fe_engine_diffusion_denoise(e._h, p(c), p(n), 5.0, p(out)) == 4
        assert flowedge_amd.last_error() == "Model has no Diffusion Policy head"
        with pytest.raises(RuntimeError):
            e.sample_condition(cond[0], x[0], np.empty(3, np.float32), steps=2)


def test_status_codes(tiny_engine, tiny):
    lib = flowedge_amd.lib()
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    out = np.empty((spec.horizon, spec.action_dim), np.float32)
    p = flowedge_amd._p
    c, n = np.ascontiguousarray(cond[0]), np.ascontiguousarray(noise[0])
    h = tiny_engine._h
    assert lib.fe_engine_sample_diffusion(h, p(c), p(n), 0, 0, 0, p(out)) == 1
    assert lib.fe_engine_sample_diffusion(h, p(c), p(n), 101, 0, 0, p(out)) == 1
    assert lib.fe_engine_sample_diffusion(h, p(c), p(n), 10, 7, 0, p(out)) == 5
    assert lib.fe_engine_sample_condition(h, p(c), p(n), 10, 0, p(out)) == 4
    assert lib.fe_engine_sample_diffusion(h, p(c), p(n), 10, 0, 0, p(out)) == 0
    assert flowedge_amd.last_error() == ""
    assert lib.fe_engine_diffusion_denoise(h, p(c), p(n), float("nan"), p(out)) == 1
    big = tiny_engine.max_batch + 1
    cb = np.zeros((big, spec.cond_dim), np.float32)
    nb = np.zeros((big, spec.horizon, spec.action_dim), np.float32)
    ob = np.empty_like(nb)
    assert lib.fe_engine_sample_diffusion_batch(h, p(cb), p(nb), big, 10, 0, 0, p(ob)) == 1
    md = tiny_engine.diffusion_metadata
    assert (md["action_dim"], md["horizon"], md["condition_dim"], md["train_timesteps"]) == (
        2, 16, 64, 100)
    assert tiny_engine.model_metadata["architecture"] == 4
    assert tiny_engine.cuda_resident


def test_reference_fixture_model(ckpt_dir):
    # The reference's own 2-stage fixture (kernel 3, groups 2, T=10, action range [-2,2]x[0,10]).
    path = unet_ref.write_fixture(os.path.join(ckpt_dir, "ref_fixture.safetensors"))
    o = oracle.Oracle(path)
    say("reference fixture model")
    with flowedge_amd.Engine(path) as e:
        sample = unet_ref.seq(8, 0.23, -0.1)
        cond = unet_ref.seq(3, 0.41, 0.2)
        assert maxerr(e.diffusion_denoise(cond, sample, 7.0), o.denoise(cond, sample, 7.0)) <= 2e-6
        cond = unet_ref.seq(3, 0.31, -0.2)
        noise = unet_ref.seq(8, 0.29, 0.1)
        ddim = e.sample_diffusion(cond, noise, steps=5)
        assert maxerr(ddim, o.sample(cond, noise, 5, 0, 1)) <= 1e-5
        ddpm = e.sample_diffusion(cond, noise, steps=5, scheduler="ddpm", seed=42)
        assert maxerr(ddpm, o.sample(cond, noise, 5, 1, 42)) <= 1e-4
        assert np.all(ddim[:, 0] >= -2) and np.all(ddim[:, 0] <= 2)
        assert np.all(ddim[:, 1] >= 0) and np.all(ddim[:, 1] <= 10)


@pytest.mark.parametrize("method,steps", [("euler", 10), ("heun", 3), ("rk4", 4)])
def test_flow_unet_small(ckpt_dir, method, steps):
    spec = ck.UNetSpec(dims=(64, 128, 256), action_dim=7, cond_dim=32, prediction=1)
    path = unet_ref.write_variant(os.path.join(ckpt_dir, "flow_small_gpu.safetensors"), spec)
    o = oracle.Oracle(path)
    cond, x0 = ck.inputs(spec, batch=3)
    say(f"flow small {method} steps={steps}")
    with flowedge_amd.Engine(path) as e:
        out = np.empty((spec.horizon, spec.action_dim), np.float32)
        e.sample_condition(cond[0], x0[0], out, steps=steps, method=method)
        want = o.sample_flow(cond[0], x0[0], steps, flowedge_amd.SOLVERS[method])
        assert maxerr(out, want) <= TOL
        batch = e.sample_condition_batch(cond, x0, steps=steps, method=method)
        assert np.array_equal(batch[0], out)
        for b in (1, 2):
            assert maxerr(batch[b], o.sample_flow(cond[b], x0[b], steps,
                                                  flowedge_amd.SOLVERS[method])) <= TOL
        with pytest.raises(RuntimeError):
            e.sample_diffusion(cond[0], x0[0])


def test_bf16_weights_small(ckpt_dir):
    spec = ck.UNetSpec(dims=(64, 128, 256), horizon=8, action_dim=14, cond_dim=96,
                       action_steps=4, bf16_weights=True)
    path = ck.write_synthetic(os.path.join(ckpt_dir, "bf16_small.safetensors"), spec)
    o = oracle.Oracle(path)
    cond, noise = ck.inputs(spec, batch=2)
    say("bf16 small")
    with flowedge_amd.Engine(path) as e:
        assert e.model_metadata["precision"] == 3
        got = e.sample_diffusion_batch(cond, noise, steps=10)
        for b in range(2):
            assert maxerr(got[b], o.sample(cond[b], noise[b], 10)) <= TOL


# ---------------------------------------------------------------------------------------------
# Full-size workloads.
# ---------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def pusht(ckpt_dir):
    return ck.cached_checkpoint("pusht", ckpt_dir)


def test_pusht_b1_ddim10_and_denoise(pusht):
    spec = ck.SPECS["pusht"]
    cond, noise = ck.inputs(spec)
    o = oracle.Oracle(pusht, threads=8)
    say("pusht B=1 DDIM-10")
    with flowedge_amd.Engine(pusht) as e:
        for t in (90.0, 0.0):
            assert maxerr(e.diffusion_denoise(cond[0], noise[0], t),
                          o.denoise(cond[0], noise[0], t)) <= 2e-5
        got = e.sample_diffusion(cond[0], noise[0], steps=10)
        err = maxerr(got, o.sample(cond[0], noise[0], 10))
        say(f"pusht DDIM-10 max err {err:.3e}")
        assert err <= TOL
        cb, nb = ck.inputs(spec, batch=3)  # below the matrix-core threshold: bit-exact
        batch = e.sample_diffusion_batch(cb, nb, steps=10)
        assert np.array_equal(batch[0], got)
        for b in range(1, 3):
            assert np.array_equal(batch[b], e.sample_diffusion(cb[b], nb[b], steps=10))


def test_pusht_kernel_paths(pusht):
    # The pusht U-Net's 29 convolutions per evaluation all have fused weight-streaming instances
    # (one sample per grid row) and matrix-core instances; the switch is the batch threshold.
    with flowedge_amd.Engine(pusht) as e:
        names = [c["name"] for c in e.convolutions()]
        assert len(names) == 29
        assert e.conv_paths(1) == ["fused"] * 29
        assert e.conv_paths(3) == ["fused"] * 29
        assert e.conv_paths(4) == ["matrix"] * 29
        assert e.conv_paths(256) == ["matrix"] * 29
        # Below the matrix-core threshold every convolution but the first (2 input channels) runs
        # with its input channels split into 8 slices.  On the matrix cores, small batches leave
        # the partial sums of a split K loop (at most 8) for the consumer to add; at 256 samples
        # the output tiles fill the GPU and nothing is split.
        assert e.conv_slices(1) == [1] + [8] * 28
        assert e.conv_slices(3) == [1] + [8] * 28
        parts = e.conv_slices(4)
        assert all(1 <= p <= 8 for p in parts) and max(parts) > 1, parts
        assert e.conv_slices(256) == [1] * 29


def test_slicing_off_matches_oracle(pusht, monkeypatch):
    # FLOWEDGE_SLICES=1 at load runs every convolution unsliced (the kernels the persistent tick
    # shares); both forms agree with the oracle.
    spec = ck.SPECS["pusht"]
    cond, noise = ck.inputs(spec, batch=2)
    o = oracle.Oracle(pusht, threads=8)
    want = [o.sample(cond[b], noise[b], 10) for b in range(2)]
    monkeypatch.setenv("FLOWEDGE_SLICES", "1")
    with flowedge_amd.Engine(pusht) as e:
        assert e.conv_slices(1) == [1] * 29
        got = e.sample_diffusion_batch(cond, noise, steps=10)
    monkeypatch.delenv("FLOWEDGE_SLICES")
    for b in range(2):
        assert maxerr(got[b], want[b]) <= TOL


def test_bimanual_bf16(ckpt_dir):
    spec = ck.SPECS["bimanual"]
    path = ck.cached_checkpoint("bimanual", ckpt_dir)
    o = oracle.Oracle(path, threads=8)
    cond, noise = ck.inputs(spec, batch=2)
    say("bimanual bf16 H=8 A=14")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_diffusion_batch(cond, noise, steps=10)
        for b in range(2):
            assert maxerr(got[b], o.sample(cond[b], noise[b], 10)) <= TOL


def test_flow_full_size(ckpt_dir):
    spec = ck.SPECS["flow"]
    path = ck.cached_checkpoint("flow", ckpt_dir)
    o = oracle.Oracle(path, threads=8)
    cond, x0 = ck.inputs(spec)
    say("flow U-Net RK4-4 and Euler-10")
    with flowedge_amd.Engine(path) as e:
        for method, steps in (("rk4", 4), ("euler", 10)):
            out = np.empty((spec.horizon, spec.action_dim), np.float32)
            e.sample_condition(cond[0], x0[0], out, steps=steps, method=method)
            want = o.sample_flow(cond[0], x0[0], steps, flowedge_amd.SOLVERS[method])
            err = maxerr(out, want)
            say(f"flow {method} max err {err:.3e}")
            assert err <= TOL


# ---------------------------------------------------------------------------------------------
# Batched path: the convolutions run as implicit GEMMs on the matrix cores (batch >= 5 / 8).
# ---------------------------------------------------------------------------------------------
def test_tiny_batched_mfma(tiny_engine, tiny_oracle):
    spec = ck.SPECS["tiny"]
    B = 19  # not a multiple of any column tile: exercises the sample masking
    cond, noise = ck.inputs(spec, batch=B)
    say(f"tiny DDIM-10 / DDPM / denoise batch={B} (matrix cores)")
    got = tiny_engine.sample_diffusion_batch(cond, noise, steps=10)
    want = tiny_oracle.sample_batch(cond, noise, 10, workers=8)
    assert maxerr(got, want) <= TOL
    got = tiny_engine.sample_diffusion_batch(cond, noise, steps=10, scheduler="ddpm", seed=7)
    want = tiny_oracle.sample_batch(cond, noise, 10, 0, 1, 7, workers=8)
    assert maxerr(got, want) <= TOL
    eps = tiny_engine.diffusion_denoise_batch(cond, noise, 50.0)
    for b in (0, 7, 18):
        assert maxerr(eps[b], tiny_oracle.denoise(cond[b], noise[b], 50.0)) <= TOL
    # Within tolerance of independent batch-1 calls (different summation order).
    for b in (0, 18):
        assert maxerr(got[b], tiny_engine.sample_diffusion(cond[b], noise[b], steps=10,
                                                           scheduler="ddpm", seed=7)) <= 2 * TOL


@pytest.mark.parametrize("workload", ["tiny", "pusht"])
def test_f32_split_matrix_core_path(ckpt_dir, monkeypatch, workload):
    # Opt-in F32 path on the BF16 matrix cores (three products of split weights and split input,
    # about 1e-5 relative per layer): held to the fp32 bound 1e-4 (measured about 7e-5 at pusht
    # size, which is why it is not the default).
    spec = ck.SPECS[workload]
    path = ck.cached_checkpoint(workload, ckpt_dir)
    B = 19 if workload == "tiny" else 16
    cond, noise = ck.inputs(spec, batch=B)
    o = oracle.Oracle(path, threads=0)
    monkeypatch.setenv("FLOWEDGE_MFMA_F32_SPLIT", "1")
    say(f"{workload} DDIM-10 batch={B} FLOWEDGE_MFMA_F32_SPLIT=1")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_diffusion_batch(cond, noise, steps=10)
        assert np.array_equal(got, e.sample_diffusion_batch(cond, noise, steps=10))
    err = maxerr(got, o.sample_batch(cond, noise, 10, workers=8))
    say(f"{workload} split batch={B} max err {err:.3e}")
    assert err <= TOL


def test_tiny_large_batch(ckpt_dir, monkeypatch):
    # A batch far above the bench sizes: large grids and per-sample offsets on the matrix-core
    # path, against the oracle on a spread of samples.
    spec = ck.SPECS["tiny"]
    path = ck.cached_checkpoint("tiny", ckpt_dir)
    B = 1000
    monkeypatch.setenv("FLOWEDGE_MAX_BATCH", "1024")
    cond, noise = ck.inputs(spec, batch=B)
    o = oracle.Oracle(path)
    say(f"tiny DDIM-10 batch={B}")
    with flowedge_amd.Engine(path) as e:
        assert e.max_batch == 1024
        got = e.sample_diffusion_batch(cond, noise, steps=10)
    idx = [0, 1, 255, 256, 511, 767, 998, 999]
    want = o.sample_batch(cond[idx], noise[idx], 10, workers=8)
    assert maxerr(got[idx], want) <= TOL
    assert np.all(np.isfinite(got))


def test_pusht_batched_mfma(pusht):
    spec = ck.SPECS["pusht"]
    B = 16
    cond, noise = ck.inputs(spec, batch=B)
    o = oracle.Oracle(pusht, threads=0)
    say(f"pusht DDIM-10 batch={B} (matrix cores)")
    with flowedge_amd.Engine(pusht) as e:
        got = e.sample_diffusion_batch(cond, noise, steps=10)
    want = o.sample_batch(cond, noise, 10, workers=8)
    err = maxerr(got, want)
    say(f"pusht batch={B} max err {err:.3e}")
    assert err <= TOL


def test_bimanual_bf16_batched_mfma(ckpt_dir):
    spec = ck.SPECS["bimanual"]
    path = ck.cached_checkpoint("bimanual", ckpt_dir)
    B = 12
    cond, noise = ck.inputs(spec, batch=B)
    o = oracle.Oracle(path, threads=0)
    say(f"bimanual bf16 DDIM-10 batch={B} (matrix cores, length-2 stage)")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_diffusion_batch(cond, noise, steps=10)
    err = maxerr(got, o.sample_batch(cond, noise, 10, workers=8))
    say(f"bimanual batch={B} max err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("bf16_mma", ["1", "0"])
def test_bf16_weights_matrix_core_paths(ckpt_dir, monkeypatch, bf16_mma):
    # BF16 weights at a batch on the matrix cores: the BF16 MFMA path (input split into two BF16
    # terms, about 2^-17 relative per product) and the F32 MFMA path (weights widened).  Both are
    # held to 1e-4 here; the contract bound for BF16-weight variants is 2e-2.
    spec = ck.UNetSpec(dims=(64, 128, 256), horizon=8, action_dim=14, cond_dim=96,
                       action_steps=4, bf16_weights=True)
    path = ck.write_synthetic(os.path.join(ckpt_dir, "bf16_small.safetensors"), spec)
    B = 8
    cond, noise = ck.inputs(spec, batch=B)
    o = oracle.Oracle(path)
    monkeypatch.setenv("FLOWEDGE_MFMA_BF16", bf16_mma)
    say(f"bf16 small batch={B} FLOWEDGE_MFMA_BF16={bf16_mma}")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_diffusion_batch(cond, noise, steps=10)
        again = e.sample_diffusion_batch(cond, noise, steps=10)
    assert np.array_equal(got, again)  # fixed summation order: repeatable
    err = maxerr(got, o.sample_batch(cond, noise, 10, workers=8))
    say(f"bf16 small batch={B} max err {err:.3e}")
    assert err <= TOL


def test_flow_batched_mfma(ckpt_dir):
    spec = ck.SPECS["flow"]
    path = ck.cached_checkpoint("flow", ckpt_dir)
    B = 9
    cond, x0 = ck.inputs(spec, batch=B)
    o = oracle.Oracle(path, threads=0)
    say(f"flow RK4-4 batch={B} (matrix cores)")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_condition_batch(cond, x0, steps=4, method="rk4")
    err = maxerr(got, o.sample_batch(cond, x0, 4, 1, flowedge_amd.SOLVERS["rk4"], workers=8))
    say(f"flow batch={B} max err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("steps", [1, 3, 10])
def test_ddpm_closed_form_constant_epsilon(ckpt_dir, steps):
    # The device DDPM step and noise stream against the float64 closed form of
    # diffusion.cc:1005-1024 on a model whose epsilon is its output bias, at batch 1 and on the
    # matrix cores (batch 9: every sample draws the same stream, as 9 independent calls).
    spec = ck.SPECS["tiny"]
    path = unet_ref.write_variant(os.path.join(ckpt_dir, "tiny_zero_out.safetensors"), spec,
                                  zero=("dp.f.o.w",))
    bias = ck.read_safetensors(path)["dp.f.o.b"]
    eps = np.tile(bias, (spec.horizon, 1))
    cond, noise = ck.inputs(spec, batch=9)
    say(f"DDPM closed form steps={steps}")
    with flowedge_amd.Engine(path) as e:
        for seed in (0, 42):
            for scale in (1.0, 0.05):
                x = noise * np.float32(scale)
                ref = unet_ref.ddpm_const_eps(x[0], eps, steps, 100, 1.0, -1.0, 1.0, seed)
                got = e.sample_diffusion(cond[0], x[0], steps=steps, scheduler="ddpm", seed=seed)
                assert maxerr(got, ref) <= 3e-5
                batch = e.sample_diffusion_batch(cond, x, steps=steps, scheduler="ddpm",
                                                 seed=seed)
                for b in (0, 4, 8):
                    want = unet_ref.ddpm_const_eps(x[b], eps, steps, 100, 1.0, -1.0, 1.0, seed)
                    assert maxerr(batch[b], want) <= 3e-5


@pytest.mark.parametrize("workload,batch", [("tiny", 1), ("tiny", 9), ("pusht", 1), ("pusht", 8)])
def test_converter_bf16_linear_layout(ckpt_dir, workload, batch):
    # The reference converter's --dtype bf16 layout: BF16 2-D linears (time MLP, FiLM), F32
    # convolutions.  Loaded through the C ABI and held to the oracle on the same file at the fp32
    # bound (the convolutions are F32; the BF16 linears are widened identically by both).
    import dataclasses
    spec = dataclasses.replace(ck.SPECS[workload], bf16_linears=True)
    path = os.path.join(ckpt_dir, f"{workload}_bf16_linears.safetensors")
    if not os.path.exists(path):
        ck.write_synthetic(path, spec)
    cond, noise = ck.inputs(spec, batch=batch)
    say(f"{workload} converter BF16-linear layout B={batch}")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_diffusion_batch(cond, noise, steps=10)
    want = oracle.Oracle(path).sample_batch(cond, noise, 10, workers=16)
    err = maxerr(got, want)
    say(f"{workload} BF16-linear layout B={batch} max err {err:.3e}")
    assert err <= TOL
