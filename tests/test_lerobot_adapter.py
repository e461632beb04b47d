"""The LeRobot deployment adapter's host logic, with stand-in engines (no GPU).

Cases follow the reference adapter's tests (integrations/lerobot/tests/test_diffusion.py:40-101):
the executed slice of the horizon, float32 contiguous forwarding, caller-owned outputs, engines
without `sample_diffusion_into`, and shape errors; plus the metadata and device checks.
"""

from __future__ import annotations

import numpy as np
import pytest

from flowedge_amd.lerobot import DiffusionActionContract, FlowEdgeDiffusionPolicy, require_device

META = {"condition_dim": 4, "action_dim": 2, "horizon": 6, "action_steps": 3,
        "observation_steps": 2}
HORIZON = np.arange(12, dtype=np.float32).reshape(6, 2)


class IntoEngine:
    """Writes a fixed horizon through sample_diffusion_into and records its arguments."""

    diffusion_metadata = META
    cuda_resident = True

    def __init__(self):
        self.calls = []

    def sample_diffusion(self, condition, noise, steps, scheduler, seed):
        raise AssertionError("the adapter must prefer sample_diffusion_into")

    def sample_diffusion_into(self, condition, noise, output, steps, scheduler, seed):
        self.calls.append((condition, noise, steps, scheduler, seed))
        output[...] = HORIZON


class ReturningEngine:
    """Has only sample_diffusion; returns the noise as the horizon."""

    diffusion_metadata = META

    def sample_diffusion(self, condition, noise, steps, scheduler, seed):
        return noise


def test_contract_executed_slice():
    c = DiffusionActionContract.from_metadata(META)
    assert (c.action_start, c.action_stop) == (1, 4)
    # pusht: horizon 16, 2 observation steps, 8 executed actions -> rows 1..8.
    c = DiffusionActionContract.from_metadata(dict(META, horizon=16, action_steps=8))
    assert (c.action_start, c.action_stop) == (1, 9)


@pytest.mark.parametrize("change,message", [
    ({"horizon": None}, "missing diffusion metadata: horizon"),
    ({"action_steps": 6}, "outside the diffusion horizon"),  # rows 1..6 of a 6-row horizon
    ({"action_dim": 0}, "positive"),
    ({"observation_steps": 0}, "observation_steps"),
])
def test_contract_rejects_bad_metadata(change, message):
    md = dict(META)
    for k, v in change.items():
        if v is None:
            del md[k]
        else:
            md[k] = v
    with pytest.raises(ValueError, match=message):
        DiffusionActionContract.from_metadata(md)


def test_chunk_forwards_float32_contiguous_and_slices():
    e = IntoEngine()
    p = FlowEdgeDiffusionPolicy(e)
    cond = np.arange(4, dtype=np.float64).reshape(1, 4)   # any shape with 4 values
    noise = np.zeros((2, 6), np.float64).T                 # float64, not C-contiguous
    chunk = p.predict_action_chunk(cond, noise, steps=7, scheduler="ddpm", seed=11)
    np.testing.assert_array_equal(chunk, HORIZON[1:4])
    c, n, steps, scheduler, seed = e.calls[0]
    for a in (c, n):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    assert c.shape == (4,) and n.shape == (6, 2)
    assert (steps, scheduler, seed) == (7, "ddpm", 11)


def test_into_writes_caller_storage():
    p = FlowEdgeDiffusionPolicy(IntoEngine())
    out = np.full((3, 2), -1.0, np.float32)
    assert p.predict_action_chunk_into(np.zeros(4), np.zeros((6, 2)), out) is out
    np.testing.assert_array_equal(out, HORIZON[1:4])
    a = np.empty(2, np.float32)
    assert p.select_action_into(np.zeros(4), np.zeros((6, 2)), a) is a
    np.testing.assert_array_equal(a, HORIZON[1])
    np.testing.assert_array_equal(p.select_action(np.zeros(4), np.zeros((6, 2))), HORIZON[1])


def test_engine_without_into_returns_horizon():
    p = FlowEdgeDiffusionPolicy(ReturningEngine())
    noise = np.arange(12, dtype=np.float32).reshape(6, 2) * 0.5
    np.testing.assert_array_equal(p.predict_action_chunk(np.zeros(4), noise), noise[1:4])


@pytest.mark.parametrize("cond,noise,kw,message", [
    (np.zeros(3), np.zeros((6, 2)), {}, "condition"),
    (np.zeros(4), np.zeros((5, 2)), {}, "noise"),
    (np.zeros(4), np.zeros(12), {}, "noise"),
    (np.zeros(4), np.zeros((6, 2)), {"steps": 0}, "steps"),
    (np.zeros(4), np.zeros((6, 2)), {"scheduler": "euler"}, "scheduler"),
])
def test_rejects_bad_arguments_before_sampling(cond, noise, kw, message):
    e = IntoEngine()
    with pytest.raises(ValueError, match=message):
        FlowEdgeDiffusionPolicy(e).predict_action_chunk(cond, noise, **kw)
    assert not e.calls


@pytest.mark.parametrize("out", [np.empty((3, 2), np.float64), np.empty((2, 3), np.float32),
                                 np.empty((3, 4), np.float32)[:, ::2]])
def test_rejects_bad_output(out):
    with pytest.raises(ValueError, match="output"):
        FlowEdgeDiffusionPolicy(IntoEngine()).predict_action_chunk_into(
            np.zeros(4), np.zeros((6, 2)), out)


def test_device_check_fails_closed():
    require_device("cuda", IntoEngine())
    require_device("cuda:0")
    with pytest.raises(RuntimeError, match="no CPU kernels"):
        require_device("cpu")
    with pytest.raises(ValueError):
        require_device("cuda:1")
    with pytest.raises(RuntimeError, match="device-resident"):
        require_device("cuda", ReturningEngine())
