"""The LeRobot adapter over the real engine: executed chunks against the CPU oracle.

Tolerance as the other fp32 parity tests: max |err| <= 1e-4 in action units.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from flowedge_amd import checkpoint as ck
from flowedge_amd.lerobot import FlowEdgeDiffusionPolicy

pytestmark = pytest.mark.gpu

TOL = 1e-4


def test_adapter_chunks_match_oracle(ckpt_dir):
    path = ck.cached_checkpoint("tiny", ckpt_dir)
    o = oracle.Oracle(path)
    spec = ck.SPECS["tiny"]
    cond, noise = ck.inputs(spec)
    print("lerobot adapter on the tiny checkpoint", flush=True)
    p = FlowEdgeDiffusionPolicy.from_checkpoint(path)
    try:
        c = p.contract
        assert (c.horizon, c.action_steps, c.observation_steps) == (16, 8, 2)
        assert p.cuda_resident
        rows = slice(c.action_start, c.action_stop)
        want = np.asarray(o.sample(cond[0], noise[0], 10, 0, 0)).reshape(16, 2)
        chunk = p.predict_action_chunk(cond[0], noise[0].reshape(16, 2))
        assert chunk.shape == (8, 2)
        assert np.max(np.abs(chunk - want[rows])) <= TOL
        action = p.select_action(cond[0], noise[0].reshape(16, 2))
        np.testing.assert_array_equal(action, chunk[0])  # same inputs, deterministic engine
        want = np.asarray(o.sample(cond[0], noise[0], 5, 1, 9)).reshape(16, 2)
        out = np.empty((8, 2), np.float32)
        p.predict_action_chunk_into(cond[0], noise[0].reshape(16, 2), out, steps=5,
                                    scheduler="ddpm", seed=9)
        assert np.max(np.abs(out - want[rows])) <= TOL
    finally:
        p.engine.close()
