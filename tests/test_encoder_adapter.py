"""CPU checks of the observation history and condition assembly (flowedge_amd.encoder), with a
stand-in image encoder: the counterpart of the reference's own tests
(integrations/lerobot/tests/test_observation.py:14-42, 63-90)."""

from __future__ import annotations

import numpy as np
import pytest

from flowedge_amd.encoder import DiffusionObservationEncoder, normalize


def make(n_obs_steps=2, **kw):
    return DiffusionObservationEncoder(
        lambda images: images.mean(axis=(1, 2, 3))[:, None], n_obs_steps,
        {"observation.state": (2,), "observation.image": (3, 2, 2)}, **kw)


def test_history_is_padded_copied_and_advanced_in_source_feature_order():
    enc = make()
    batch = {"observation.state": np.array([[1.0, 2.0]]),
             "observation.image": np.ones((1, 3, 2, 2))}
    enc.observe(batch, normalized=True)
    np.testing.assert_array_equal(enc.condition(), [1, 2, 1, 1, 2, 1])
    batch["observation.state"].fill(3)   # the recorded frame is a copy
    batch["observation.image"].fill(4)
    enc.observe(batch, normalized=True)
    np.testing.assert_array_equal(enc.condition(), [1, 2, 1, 3, 3, 4])
    enc.reset()
    with pytest.raises(ValueError):
        enc.condition()


def test_environment_state_and_cameras_follow_the_image_features():
    enc = DiffusionObservationEncoder(
        lambda images: images.reshape(len(images), -1)[:, :1], 1,
        {"observation.state": (1,), "a": (1, 1, 1), "b": (1, 1, 1), "env": (2,)},
        image_keys=("a", "b"), env_state_key="env")
    enc.observe({"observation.state": [[5.0]], "a": [[[[6.0]]]], "b": [[[[7.0]]]],
                 "env": [[8.0, 9.0]]}, normalized=True)
    np.testing.assert_array_equal(enc.condition(), [5, 6, 7, 8, 9])


def test_observe_rejects_bad_shapes_and_non_finite_values():
    enc = make()
    with pytest.raises(ValueError, match="shape"):
        enc.observe({"observation.state": np.zeros((1, 3)),
                     "observation.image": np.zeros((1, 3, 2, 2))}, normalized=True)
    with pytest.raises(ValueError, match="non-finite"):
        enc.observe({"observation.state": np.array([[np.nan, 0.0]]),
                     "observation.image": np.zeros((1, 3, 2, 2))}, normalized=True)
    with pytest.raises(ValueError):
        make(n_obs_steps=0)


def test_normalization_matches_lerobot_modes():
    # min_max to [-1, 1] (test_observation.py:63-90: min 0, max 10, [0, 10] -> [-1, 1]).
    got = normalize([[0.0, 10.0]], {"min": np.zeros(2), "max": np.full(2, 10.0)}, "min_max")
    np.testing.assert_allclose(got, [[-1.0, 1.0]], atol=1e-6)
    got = normalize([[3.0]], {"mean": [1.0], "std": [2.0]}, "mean_std")
    np.testing.assert_allclose(got, [[1.0]], atol=1e-6)
    enc = make(normalization={"observation.state": ("min_max", {"min": [0, 0], "max": [10, 10]})})
    enc.observe({"observation.state": np.array([[0.0, 10.0]]),
                 "observation.image": np.ones((1, 3, 2, 2))})
    np.testing.assert_allclose(enc.condition(), [-1, 1, 1, -1, 1, 1], atol=1e-6)
