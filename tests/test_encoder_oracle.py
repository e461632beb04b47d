"""CPU pins of the observation-encoder oracle (oracle/encoder_ref.py).

Each operation is held to an independent implementation: brute-force loops or torch's float64
functional ops; spatial softmax to its closed forms; the whole encoder to a torch float64 build
from ``nn`` layers wired as torchvision's resnet18 BasicBlocks; the condition layout to the
reference's own test vectors (integrations/lerobot/tests/test_observation.py:14-42).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from flowedge_amd import checkpoint as ck
from oracle import encoder_ref as er


def rng(seed=0):
    return np.random.default_rng(seed)


def test_conv2d_matches_brute_force():
    r = rng(1)
    x = r.standard_normal((3, 7, 6))
    w = r.standard_normal((4, 3, 3, 3))
    for stride, pad in ((1, 1), (2, 1), (2, 0), (1, 0)):
        got = er.conv2d(x, w, stride, pad)
        xp = np.pad(x, ((0, 0), (pad, pad), (pad, pad)))
        ho = (xp.shape[1] - 3) // stride + 1
        wo = (xp.shape[2] - 3) // stride + 1
        want = np.zeros((4, ho, wo))
        for o in range(4):
            for i in range(ho):
                for j in range(wo):
                    want[o, i, j] = np.sum(
                        xp[:, i * stride:i * stride + 3, j * stride:j * stride + 3] * w[o])
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("k,stride,pad", [(7, 2, 3), (3, 1, 1), (3, 2, 1), (1, 2, 0), (1, 1, 0)])
def test_conv2d_matches_torch(k, stride, pad):
    r = rng(2)
    x = r.standard_normal((5, 13, 11))
    w = r.standard_normal((6, 5, k, k))
    b = r.standard_normal(6)
    got = er.conv2d(x, w, stride, pad, b)
    want = F.conv2d(torch.from_numpy(x)[None], torch.from_numpy(w), torch.from_numpy(b),
                    stride=stride, padding=pad)[0].numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_group_norm_and_max_pool_match_torch():
    r = rng(3)
    x = r.standard_normal((32, 9, 7)) * 3 + 1
    g = r.standard_normal(32)
    b = r.standard_normal(32)
    want = F.group_norm(torch.from_numpy(x)[None], 2, torch.from_numpy(g), torch.from_numpy(b),
                        eps=1e-5)[0].numpy()
    np.testing.assert_allclose(er.group_norm(x, g, b, 2), want, rtol=1e-12, atol=1e-12)
    for shape in ((4, 42, 42), (3, 21, 20), (2, 5, 6)):
        y = r.standard_normal(shape)
        want = F.max_pool2d(torch.from_numpy(y)[None], 3, 2, 1)[0].numpy()
        np.testing.assert_array_equal(er.max_pool(y), want)


def test_spatial_softmax_closed_forms():
    r = rng(4)
    x = r.standard_normal((8, 3, 5))
    # Zero 1x1 conv: uniform attention, expected position the grid's mean (0, 0).
    kp = er.spatial_softmax(x, np.zeros((4, 8, 1, 1)), np.zeros(4))
    np.testing.assert_allclose(kp, 0.0, atol=1e-15)
    # One dominant position: the keypoint is that grid point (x along the width, y down).
    xs = np.zeros((1, 3, 5))
    xs[0, 2, 1] = 1e3
    kp = er.spatial_softmax(xs, np.ones((1, 1, 1, 1)), np.zeros(1))
    np.testing.assert_allclose(kp[0], [np.linspace(-1, 1, 5)[1], 1.0], atol=1e-12)
    # A constant added to every position of a map changes nothing (softmax shift invariance).
    w = r.standard_normal((3, 8, 1, 1))
    b = r.standard_normal(3)
    np.testing.assert_allclose(er.spatial_softmax(x, w, b), er.spatial_softmax(x, w, b + 7.0),
                               atol=1e-13)


def test_center_crop_box():
    # torchvision CenterCrop: int(round((size - crop) / 2)), Python rounding (half to even).
    assert er.center_crop_box(96, 96, 84, 84) == (6, 6)
    assert er.center_crop_box(97, 85, 84, 84) == (6, 0)
    assert er.center_crop_box(99, 84, 84, 84) == (8, 0)


def test_condition_layout_matches_reference_vectors():
    # integrations/lerobot/tests/test_observation.py:14-42: two steps of state [1, 2] and a
    # one-value image feature 1, then a new step with state [3, 3] and feature 4.
    np.testing.assert_array_equal(er.condition([[1, 2], [1, 2]], [[1], [1]]), [1, 2, 1, 1, 2, 1])
    np.testing.assert_array_equal(er.condition([[1, 2], [3, 3]], [[1], [4]]), [1, 2, 1, 3, 3, 4])
    np.testing.assert_array_equal(er.condition([[1], [2]], [[3], [4]], [[5], [6]]),
                                  [1, 3, 5, 2, 4, 6])


class _Block(torch.nn.Module):
    """torchvision BasicBlock with GroupNorm(C/16), built from nn layers."""

    def __init__(self, t, p, cin, cout, stride):
        super().__init__()
        self.c1 = torch.nn.Conv2d(cin, cout, 3, stride, 1, bias=False)
        self.n1 = torch.nn.GroupNorm(cout // 16, cout)
        self.c2 = torch.nn.Conv2d(cout, cout, 3, 1, 1, bias=False)
        self.n2 = torch.nn.GroupNorm(cout // 16, cout)
        self.ds = None
        if p + "downsample.0.weight" in t:
            self.ds = torch.nn.Sequential(torch.nn.Conv2d(cin, cout, 1, stride, bias=False),
                                          torch.nn.GroupNorm(cout // 16, cout))
        with torch.no_grad():
            self.c1.weight.copy_(t[p + "conv1.weight"])
            self.n1.weight.copy_(t[p + "bn1.weight"])
            self.n1.bias.copy_(t[p + "bn1.bias"])
            self.c2.weight.copy_(t[p + "conv2.weight"])
            self.n2.weight.copy_(t[p + "bn2.weight"])
            self.n2.bias.copy_(t[p + "bn2.bias"])
            if self.ds is not None:
                self.ds[0].weight.copy_(t[p + "downsample.0.weight"])
                self.ds[1].weight.copy_(t[p + "downsample.1.weight"])
                self.ds[1].bias.copy_(t[p + "downsample.1.bias"])

    def forward(self, x):
        h = torch.relu(self.n1(self.c1(x)))
        h = self.n2(self.c2(h))
        return torch.relu(h + (x if self.ds is None else self.ds(x)))


def torch_encoder(t: dict, image: np.ndarray, crop) -> np.ndarray:
    tt = {k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in t.items()}
    layers = [torch.nn.Conv2d(3, 64, 7, 2, 3, bias=False), torch.nn.GroupNorm(4, 64),
              torch.nn.ReLU(), torch.nn.MaxPool2d(3, 2, 1)]
    with torch.no_grad():
        layers[0].weight.copy_(tt["backbone.0.weight"])
        layers[1].weight.copy_(tt["backbone.1.weight"])
        layers[1].bias.copy_(tt["backbone.1.bias"])
    cin = 64
    for s, cout in enumerate((64, 128, 256, 512)):
        for blk in range(2):
            layers.append(_Block(tt, f"backbone.{4 + s}.{blk}.", cin if blk == 0 else cout, cout,
                                 2 if (s > 0 and blk == 0) else 1))
        cin = cout
    net = torch.nn.Sequential(*layers).double()
    x = torch.from_numpy(np.asarray(image, np.float64))
    if crop is not None:
        top, left = er.center_crop_box(x.shape[1], x.shape[2], *crop)
        x = x[:, top:top + crop[0], left:left + crop[1]]
    with torch.no_grad():
        fmap = net(x[None])[0]
        logits = F.conv2d(fmap[None], tt["pool.nets.weight"], tt["pool.nets.bias"])[0]
        k, h, w = logits.shape
        att = torch.softmax(logits.reshape(k, h * w), dim=-1)
        kp = att @ tt["pool.pos_grid"]
        return torch.relu(F.linear(kp.reshape(-1), tt["out.weight"], tt["out.bias"])).numpy()


def test_encoder_matches_torch_build():
    spec = ck.EncoderSpec()
    t = {k[len(ck.ENCODER_PREFIX):]: v for k, v in ck.synthetic_encoder_tensors(spec)}
    images = ck.encoder_images(spec, 2)
    for img in images:
        got = er.encode(t, img, spec.crop_hw)
        want = torch_encoder(t, img, spec.crop_hw)
        assert got.shape == (64,)
        np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-11)
    # The synthetic position buffer is the grid the encoder uses.
    h, w = spec.feature_map_hw()
    px, py = np.meshgrid(np.linspace(-1, 1, w), np.linspace(-1, 1, h))
    np.testing.assert_allclose(t["pool.pos_grid"], np.stack([px.ravel(), py.ravel()], 1),
                               atol=1e-7)
