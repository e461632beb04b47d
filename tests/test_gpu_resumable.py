"""GPU tests of the resumable solves (engine.h:321-366 and the DDIM/DDPM counterpart).

Parity bar: after k of n steps the action equals the oracle's first k steps within 1e-4 (action
units, the same tolerance as whole samples); after all n steps it equals the one-call sample of
the same engine bit for bit (the same batch-1 kernels with the same arguments run in the same
order).  Status codes and messages follow engine.cc:585-720 and engine_runtime.cc:494-561.
"""

from __future__ import annotations

import ctypes
import os
import time

import numpy as np
import pytest

import flowedge_amd
import oracle
from flowedge_amd import checkpoint as ck
from oracle import fingerprint
from tests import unet_ref

pytestmark = pytest.mark.gpu

TOL = 1e-4
RUNNING, COMPLETE, CANCELLED, FAILED = 0, 1, 2, 3


def say(msg: str):
    print(msg, flush=True)


def maxerr(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


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


FLOW_SPEC = ck.UNetSpec(dims=(64, 128, 256), action_dim=7, cond_dim=32, prediction=1)


@pytest.fixture(scope="module")
def flow_small(ckpt_dir):
    return unet_ref.write_variant(os.path.join(ckpt_dir, "flow_small_resume.safetensors"),
                                  FLOW_SPEC)


def _advance(lib_fn, engine, budget, out):
    rem = ctypes.c_size_t(12345)
    rc = lib_fn(engine._h, budget, flowedge_amd._p(out), ctypes.byref(rem))
    return rc, int(rem.value)


@pytest.mark.parametrize("scheduler,seed", [("ddim", 0), ("ddpm", 42)])
def test_diffusion_resumable_matches_oracle_and_sample(tiny_engine, tiny_oracle, scheduler, seed):
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    steps = 10
    say(f"tiny resumable {scheduler} seed={seed}")
    tiny_engine.diffusion_begin(cond[0], noise[0], steps=steps, scheduler=scheduler, seed=seed)
    md = tiny_engine.flow_metadata
    assert (md["status"], md["remaining_nfe"], md["solver"]) == (
        RUNNING, steps, flowedge_amd.SCHEDULERS[scheduler])
    out = np.empty((spec.horizon, spec.action_dim), np.float32)
    done = 0
    for budget in (3, 1, 4, 5):
        remaining = tiny_engine.diffusion_advance(out, budget)
        done = min(steps, done + budget)
        assert remaining == steps - done
        want = tiny_oracle.sample_partial(cond[0], noise[0], steps, done,
                                          flowedge_amd.SCHEDULERS[scheduler], seed)
        assert maxerr(out, want) <= TOL, f"after {done} steps"
    assert tiny_engine.flow_metadata["status"] == COMPLETE
    assert tiny_engine.flow_metadata["remaining_nfe"] == 0
    whole = tiny_engine.sample_diffusion(cond[0], noise[0], steps=steps, scheduler=scheduler,
                                         seed=seed)
    assert np.array_equal(out, whole)


def test_diffusion_resumable_complete_solve_stays_readable(tiny_engine):
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    tiny_engine.diffusion_begin(cond[0], noise[0], steps=3)
    out = np.empty((spec.horizon, spec.action_dim), np.float32)
    assert tiny_engine.diffusion_advance(out, 100) == 0
    again = np.zeros_like(out)
    assert tiny_engine.diffusion_advance(again, 1) == 0  # flow.cc:266: nothing left to run
    assert np.array_equal(out, again)


def test_flow_resumable_matches_oracle_and_sample(flow_small):
    o = oracle.Oracle(flow_small)
    cond, x0 = ck.inputs(FLOW_SPEC)
    out = np.empty((FLOW_SPEC.horizon, FLOW_SPEC.action_dim), np.float32)
    with flowedge_amd.Engine(flow_small) as e:
        for method, steps in (("rk4", 4), ("heun", 3), ("euler", 5)):
            say(f"flow resumable {method} steps={steps}")
            m = flowedge_amd.SOLVERS[method]
            per = {"euler": 1, "heun": 2, "rk4": 4}[method]
            e.flow_begin(cond[0], x0[0], steps=steps, method=method)
            for k in range(1, steps + 1):
                assert e.flow_advance(out, 1) == steps - k
                assert maxerr(out, o.sample_flow_partial(cond[0], x0[0], steps, m, k)) <= TOL
                md = e.flow_metadata
                assert md["remaining_nfe"] == (steps - k) * per
                assert md["status"] == (COMPLETE if k == steps else RUNNING)
                assert md["solver"] == m
            whole = np.empty_like(out)
            e.sample_condition(cond[0], x0[0], whole, steps=steps, method=method)
            assert np.array_equal(out, whole)


def test_flow_time_tables_across_pool_reset(flow_small):
    # One-shot flow calls keep their FiLM time rows per (steps, method) in a 256-row pool; a call
    # whose rows no longer fit starts the pool over and drops the graphs that read it.  Resumable
    # solves compute their rows themselves, so each one-shot call must equal the stepped solve.
    cond, x0 = ck.inputs(FLOW_SPEC)
    shape = (FLOW_SPEC.horizon, FLOW_SPEC.action_dim)
    with flowedge_amd.Engine(flow_small) as e:
        def whole(method, steps):
            out = np.empty(shape, np.float32)
            e.sample_condition(cond[0], x0[0], out, steps=steps, method=method)
            return out

        def stepped(method, steps):
            out = np.empty(shape, np.float32)
            e.flow_begin(cond[0], x0[0], steps=steps, method=method)
            assert e.flow_advance(out, steps) == 0
            return out

        first = whole("rk4", 4)
        assert np.array_equal(first, stepped("rk4", 4))
        for steps in (20, 21, 22, 23):  # 16 + 80 + 84 + 88 rows > 256: the pool starts over
            say(f"flow rk4-{steps} one-shot vs stepped")
            assert np.array_equal(whole("rk4", steps), stepped("rk4", steps))
        assert np.array_equal(whole("rk4", 4), first)
        assert np.array_equal(whole("euler", 10), stepped("euler", 10))


def test_model_digest_matches_reference_fingerprint(tiny, tiny_engine, flow_small):
    want = fingerprint.fingerprint(tiny)
    assert tiny_engine.model_metadata["model_digest"] == want
    assert flowedge_amd.weights_digest(tiny) == want
    with flowedge_amd.Engine(flow_small) as e:
        assert e.model_metadata["model_digest"] == fingerprint.fingerprint(flow_small)
        assert e.model_metadata["model_digest"] != want


def test_flow_request_cancellation(flow_small):
    lib = flowedge_amd.lib()
    cond, x0 = ck.inputs(FLOW_SPEC)
    out = np.empty((FLOW_SPEC.horizon, FLOW_SPEC.action_dim), np.float32)
    with flowedge_amd.Engine(flow_small) as e:
        say("flow request cancellation")
        e.flow_begin(cond[0], x0[0], steps=4, method="euler", generation=5, timestamp_ns=100,
                     deadline_ns=200)
        md = e.flow_metadata
        assert (md["generation"], md["timestamp_ns"], md["deadline_ns"]) == (5, 100, 200)
        assert md["model_digest"] == e.model_metadata["model_digest"]
        assert e.flow_advance(out, 1) == 3
        partial = out.copy()
        e.cancel_before(5)  # not newer: keeps running
        assert e.flow_advance(out, 1) == 2
        e.cancel_before(6)
        rc, rem = _advance(lib.fe_engine_flow_advance, e, 2, out)
        assert (rc, rem) == (8, 2)
        assert flowedge_amd.last_error() == "Flow solve was cancelled by a newer generation"
        assert e.flow_metadata["status"] == CANCELLED
        rc, rem = _advance(lib.fe_engine_flow_advance, e, 1, out)
        assert (rc, rem) == (8, 2)
        assert not np.array_equal(out, partial)  # the state after 2 steps was copied out
        # A request older than the latest generation is cancelled before its first step.
        e.flow_begin(cond[0], x0[0], steps=4, method="euler", generation=4)
        rc, rem = _advance(lib.fe_engine_flow_advance, e, 1, out)
        assert (rc, rem) == (8, 4)
        # A newer one runs; an untracked solve ignores cancellation.
        e.flow_begin(cond[0], x0[0], steps=4, method="euler", generation=7)
        assert e.flow_advance(out, 4) == 0
        e.flow_begin(cond[0], x0[0], steps=2, method="euler")
        e.cancel_before(1000)
        assert e.flow_advance(out, 2) == 0
        assert e.flow_metadata["status"] == COMPLETE


def test_diffusion_generation_cancellation(tiny_engine):
    lib = flowedge_amd.lib()
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    out = np.empty((spec.horizon, spec.action_dim), np.float32)
    c, n = np.ascontiguousarray(cond[0]), np.ascontiguousarray(noise[0])
    p = flowedge_amd._p
    h = tiny_engine._h
    base = 1 << 40  # above anything earlier tests announced on this engine
    assert lib.fe_engine_diffusion_begin_generation(h, p(c), p(n), 10, 0, 0, base) == 0
    assert _advance(lib.fe_engine_diffusion_advance, tiny_engine, 2, out) == (0, 8)
    tiny_engine.cancel_before(base + 1)
    assert _advance(lib.fe_engine_diffusion_advance, tiny_engine, 2, out) == (8, 8)
    assert flowedge_amd.last_error() == "Diffusion solve was cancelled by a newer generation"


def test_resumable_status_codes(tiny_engine, flow_small):
    lib = flowedge_amd.lib()
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    out = np.empty((spec.horizon, spec.action_dim), np.float32)
    p = flowedge_amd._p
    c, n = np.ascontiguousarray(cond[0]), np.ascontiguousarray(noise[0])
    h = tiny_engine._h
    # Epsilon model: no flow head (engine_runtime.cc:505-508).
    assert lib.fe_engine_flow_begin(h, p(c), p(n), 4, 0) == 4
    assert flowedge_amd.last_error() == "Model has no flow head to sample from"
    assert lib.fe_engine_flow_begin(h, p(c), p(n), 4, 9) == 5
    assert lib.fe_engine_flow_begin(h, p(c), p(n), 0, 0) == 1
    assert lib.fe_engine_diffusion_begin(h, p(c), p(n), 101, 0, 0) == 1
    assert lib.fe_engine_diffusion_begin(h, p(c), p(n), 10, 3, 0) == 5
    # Another sampling call ends the solve: its buffers are reused.
    tiny_engine.diffusion_begin(c, n, steps=10)
    tiny_engine.sample_diffusion(c, n, steps=10)
    assert _advance(lib.fe_engine_diffusion_advance, tiny_engine, 1, out)[0] == 6
    assert flowedge_amd.last_error() == "No resumable diffusion sample is active"
    assert tiny_engine.flow_metadata["status"] == FAILED
    assert _advance(lib.fe_engine_flow_advance, tiny_engine, 1, out)[0] == 6
    assert flowedge_amd.last_error() == "No resumable flow sample is active"
    assert _advance(lib.fe_engine_diffusion_advance, tiny_engine, 0, out)[0] == 1
    # Versioned request metadata (engine.cc:601-669).
    md = flowedge_amd.ConditionMetadata()
    assert lib.fe_engine_make_condition_metadata(h, 10, 5, 1, 4, 0, ctypes.byref(md)) == 1
    assert lib.fe_engine_make_condition_metadata(h, 10, 0, 1, 4, 7, ctypes.byref(md)) == 5
    with flowedge_amd.Engine(flow_small) as e:
        fc, fx = ck.inputs(FLOW_SPEC)
        fc, fx = np.ascontiguousarray(fc[0]), np.ascontiguousarray(fx[0])
        assert lib.fe_engine_make_condition_metadata(e._h, 10, 20, 3, 4, 2,
                                                     ctypes.byref(md)) == 0
        assert (md.struct_size, md.protocol_version, md.solver) == (ctypes.sizeof(md), 1, 2)
        assert (md.solver_steps, md.remaining_nfe) == (4, 16)
        assert (md.condition_dim, md.action_dim) == (FLOW_SPEC.cond_dim, FLOW_SPEC.action_dim)
        assert bytes(md.model_digest).hex() == e.model_metadata["model_digest"]
        good = bytes(md)

        def request(mutate) -> int:
            m = flowedge_amd.ConditionMetadata.from_buffer_copy(good)
            mutate(m)
            return lib.fe_engine_flow_begin_request(e._h, p(fc), p(fx), ctypes.byref(m))

        assert request(lambda m: None) == 0
        assert request(lambda m: setattr(m, "protocol_version", 2)) == 1
        assert request(lambda m: setattr(m, "reserved", 1)) == 1
        assert request(lambda m: setattr(m, "struct_size", 8)) == 1
        assert request(lambda m: setattr(m, "solver", 3)) == 5
        assert request(lambda m: setattr(m, "remaining_nfe", 15)) == 9
        assert request(lambda m: setattr(m, "action_dim", 6)) == 9

        def flip_digest(m):
            m.model_digest[0] ^= 0x80

        assert request(flip_digest) == 9
        assert flowedge_amd.last_error() == "Flow request metadata is incompatible with this model"
        # Velocity model: no DDIM/DDPM solve.
        assert lib.fe_engine_diffusion_begin(e._h, p(fc), p(fx), 10, 0, 0) == 4


def test_pusht_resumable_one_step_per_call(ckpt_dir):
    spec = ck.SPECS["pusht"]
    path = ck.cached_checkpoint("pusht", ckpt_dir)
    cond, noise = ck.inputs(spec)
    out = np.empty((spec.horizon, spec.action_dim), np.float32)
    with flowedge_amd.Engine(path) as e:
        say("pusht resumable DDIM-10, one step per call")
        whole = e.sample_diffusion(cond[0], noise[0], steps=10)
        e.diffusion_begin(cond[0], noise[0], steps=10)
        times = []
        for k in range(10):
            t0 = time.perf_counter()
            assert e.diffusion_advance(out, 1) == 9 - k
            times.append(time.perf_counter() - t0)
        assert np.array_equal(out, whole)
        say(f"pusht advance(1) host-to-host: median {1e3 * np.median(times):.3f} ms")
