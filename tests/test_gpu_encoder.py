"""The HIP observation encoder against the float64 oracle (oracle/encoder_ref.py), through the
C ABI (fe_encoder_*).

Synthetic LeRobot-named encoder weights (resnet18 + GroupNorm, 32 keypoints), pusht camera size
96 x 96 center-cropped to 84 x 84.  Features are ReLU outputs of order 0.1-1; the bound is the
fp32 one of the condition, 1e-4.  End to end, images + state -> condition -> DDIM-10 action of the
pusht-size head is held to the oracle's chain (encoder_ref + the Diffusion Policy oracle).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch  # before the library's first HIP call, as the other GPU suites import it

import flowedge_amd
import oracle
from flowedge_amd import checkpoint as ck
from flowedge_amd.encoder import DiffusionObservationEncoder, RgbEncoder
from oracle import encoder_ref as er

pytestmark = pytest.mark.gpu

TOL = 1e-4


def say(msg: str):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def enc_path(ckpt_dir):
    return ck.cached_encoder(ckpt_dir)


def oracle_tensors(path):
    t = ck.read_safetensors(path)
    return {k[len(ck.ENCODER_PREFIX):]: v for k, v in t.items() if k.startswith(ck.ENCODER_PREFIX)}


@pytest.mark.parametrize("n", [1, 2, 3])
def test_encoder_matches_oracle(enc_path, n):
    spec = ck.EncoderSpec()
    images = ck.encoder_images(spec, n, seed=5 + n)
    t = oracle_tensors(enc_path)
    with RgbEncoder(enc_path) as e:
        assert (e.channels, e.feature_dim, e.keypoints) == (3, 64, 32)
        say(f"encoder n={n}")
        got = e.encode(images)
        say(f"encoder n={n}: {e.last_device_ms:.3f} ms")
    for i in range(n):
        want = er.encode(t, images[i], spec.crop_hw)
        err = float(np.abs(got[i] - want).max())
        say(f"image {i}: max |err| {err:.3e} (max |feature| {np.abs(want).max():.3f})")
        assert err <= TOL


@pytest.mark.parametrize("image_hw,crop_hw", [((120, 160), None), ((97, 85), (84, 84))])
def test_encoder_other_geometries(tmp_path, image_hw, crop_hw):
    # A wide camera without a crop (odd feature-map sizes through every stride-2 stage: 60x80,
    # 30x40, 15x20, 8x10, 4x5) and odd crop margins (torchvision rounds 6.5 down to 6, 0.5 to 0).
    spec = ck.EncoderSpec(image_hw=image_hw, crop_hw=crop_hw)
    path = str(tmp_path / "enc.safetensors")
    ck.write_safetensors(path, ck.synthetic_encoder_tensors(spec))
    images = ck.encoder_images(spec, 2, seed=13)
    t = oracle_tensors(path)
    with RgbEncoder(path, image_hw=image_hw, crop_hw=crop_hw, max_images=2) as e:
        got = e.encode(images)
    for i in range(2):
        want = er.encode(t, images[i], crop_hw)
        err = float(np.abs(got[i] - want).max())
        say(f"{image_hw} crop {crop_hw} image {i}: max |err| {err:.3e}")
        assert err <= TOL


def test_encoder_largest_image_count(enc_path):
    # 64 images (the most one call takes): no split reduction at this count, the workspace
    # planned for it; the first, a middle and the last image against the oracle.
    spec = ck.EncoderSpec()
    images = ck.encoder_images(spec, 64, seed=17)
    t = oracle_tensors(enc_path)
    with RgbEncoder(enc_path, max_images=64) as e:
        got = e.encode(images)
        say(f"encoder n=64: {e.last_device_ms:.3f} ms, arena {e.device_bytes / 2**20:.1f} MiB")
    for i in (0, 31, 63):
        want = er.encode(t, images[i], spec.crop_hw)
        err = float(np.abs(got[i] - want).max())
        say(f"image {i}: max |err| {err:.3e}")
        assert err <= TOL


def test_encoder_device_output_lands_in_condition_layout(enc_path):
    spec = ck.EncoderSpec()
    images = ck.encoder_images(spec, 2, seed=11)
    dev = torch.device("cuda:0")
    with RgbEncoder(enc_path) as e:
        host = e.encode(images)
        d_img = torch.from_numpy(images).to(dev)
        # Condition layout of two steps: [state (2), features (64)] per step.
        cond = torch.full((2, 66), -7.0, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        e.encode_device(d_img.data_ptr(), 2, cond.data_ptr(), 66, 2)
        c = cond.cpu().numpy()
    np.testing.assert_array_equal(c[:, :2], -7.0)   # the state slots are left alone
    np.testing.assert_array_equal(c[:, 2:], host)   # same graph, same bits


def test_observation_to_action_matches_oracle(enc_path, ckpt_dir):
    spec = ck.EncoderSpec()
    head = ck.cached_checkpoint("pusht", ckpt_dir)
    t = oracle_tensors(enc_path)
    images = ck.encoder_images(spec, 2, seed=21)
    states = np.array([[0.25, -0.5], [0.3, -0.4]], np.float32)
    features = {"observation.state": (2,), "observation.image": (3, 96, 96)}
    noise = ck.gaussian(2, 32).reshape(16, 2)
    with RgbEncoder(enc_path) as e, flowedge_amd.Engine(head) as eng:
        obs = DiffusionObservationEncoder(e, 2, features)
        for s in range(2):
            obs.observe({"observation.state": states[s:s + 1],
                         "observation.image": images[s:s + 1]}, normalized=True)
        cond = obs.condition()
        assert cond.shape == (132,)
        action = eng.sample_diffusion(cond, noise, steps=10)
    want_cond = er.condition(states, np.stack([er.encode(t, images[s], spec.crop_hw)
                                               for s in range(2)]))
    assert float(np.abs(cond - want_cond).max()) <= TOL
    o = oracle.Oracle(head, threads=8)
    want = o.sample(want_cond.astype(np.float32), noise, 10)
    err = float(np.abs(action - want).max())
    say(f"observation -> DDIM-10 action: max |err| {err:.3e}")
    assert err <= TOL


def test_encoder_load_errors(ckpt_dir, tmp_path):
    spec = ck.EncoderSpec()
    tensors = dict(ck.synthetic_encoder_tensors(spec))
    del tensors[ck.ENCODER_PREFIX + "backbone.6.1.conv2.weight"]
    bad = str(tmp_path / "missing.safetensors")
    ck.write_safetensors(bad, tensors.items())
    with pytest.raises(RuntimeError, match="backbone.6.1.conv2.weight"):
        RgbEncoder(bad)
    path = ck.cached_encoder(ckpt_dir)
    with pytest.raises(RuntimeError, match="Missing"):
        RgbEncoder(path, prefix="policy.")
    with pytest.raises(RuntimeError, match="Invalid"):
        RgbEncoder(path, crop_hw=(100, 84))
    with RgbEncoder(path) as e:
        with pytest.raises(ValueError):
            e.encode(np.zeros((1, 3, 84, 84), np.float32))
        with pytest.raises(RuntimeError, match="non-finite"):
            e.encode(np.full((1, 3, 96, 96), np.nan, np.float32))
        with pytest.raises(RuntimeError, match="Invalid"):
            e.encode(np.zeros((9, 3, 96, 96), np.float32))
