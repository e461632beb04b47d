"""Float64 numpy restatement of the Diffusion Policy observation encoder — test infrastructure only.

Imported only by ``tests/`` (as the checker of the HIP encoder), never by the library.

The reference runs LeRobot's ``DiffusionRgbEncoder`` through torch to turn camera images into the
head's condition vector (``integrations/lerobot/src/flowedge_lerobot/observation.py:152-216``):
``condition()`` stacks, per observation step, the state, the image features and the optional
environment state, and flattens them.  LeRobot (an absent dependency of the reference, published
module ``lerobot/policies/diffusion/modeling_diffusion.py``) defines the encoder as

- a center crop to ``crop_shape`` in evaluation (torchvision ``CenterCrop``: top =
  round((H - h) / 2), left = round((W - w) / 2));
- torchvision ``resnet18`` without its average pool and fc layer, every ``BatchNorm2d`` replaced
  by ``GroupNorm(num_features // 16, num_features)`` (``use_group_norm``): a 7x7 stride-2 stem
  conv (pad 3, no bias), GN, ReLU, 3x3 stride-2 max pool (pad 1), then four stages of two
  ``BasicBlock``s (3x3 convs, pad 1, no bias; the first block of stages 2-4 has stride 2 and a
  1x1 stride-2 conv + GN on the identity path): ``relu(gn2(conv2(relu(gn1(conv1(x))))) + id)``;
- ``SpatialSoftmax``: a 1x1 conv to ``num_kp`` keypoint maps, a softmax over the H*W positions of
  each, and the expected (x, y) under it on the grid ``np.meshgrid(linspace(-1, 1, W),
  linspace(-1, 1, H))`` (x along the width), flattened as [kp0_x, kp0_y, kp1_x, ...];
- ``out``: Linear(2 num_kp, 2 num_kp) followed by ReLU.

Tensor names follow LeRobot's state dict under ``diffusion.rgb_encoder.``: ``backbone.0`` stem
conv, ``backbone.1`` stem GN, ``backbone.{4..7}.{0,1}.{conv1,bn1,conv2,bn2}`` blocks,
``backbone.{5..7}.0.downsample.{0,1}`` projections, ``pool.nets``, ``out``.

Pins (``tests/test_encoder_oracle.py``): conv2d against brute force and torch ``F.conv2d``, group
norm against ``F.group_norm``, max pool against ``F.max_pool2d`` (all float64), spatial softmax
against closed forms (uniform maps give (0, 0), one dominant position gives its grid point), the
whole encoder against an independent torch float64 build from ``nn`` layers, and the condition
layout against the reference's own test vectors
(``integrations/lerobot/tests/test_observation.py:14-42``).
"""

from __future__ import annotations

import numpy as np

STAGES = (64, 128, 256, 512)  # resnet18 stage widths
BLOCKS = 2                    # BasicBlocks per stage


def center_crop_box(height: int, width: int, crop_h: int, crop_w: int) -> tuple[int, int]:
    """(top, left) of torchvision's center crop (it rounds (size - crop) / 2 half to even)."""
    return int(round((height - crop_h) / 2.0)), int(round((width - crop_w) / 2.0))


def conv2d(x: np.ndarray, w: np.ndarray, stride: int = 1, pad: int = 0,
           b: np.ndarray | None = None) -> np.ndarray:
    """Cross-correlation of x [C][H][W] with w [O][C][kh][kw] (zero padding), float64."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    o, c, kh, kw = w.shape
    xp = np.pad(x, ((0, 0), (pad, pad), (pad, pad)))
    hout = (xp.shape[1] - kh) // stride + 1
    wout = (xp.shape[2] - kw) // stride + 1
    win = np.lib.stride_tricks.sliding_window_view(xp, (kh, kw), axis=(1, 2))
    win = win[:, ::stride, ::stride][:, :hout, :wout]  # [C][Ho][Wo][kh][kw]
    y = np.einsum("chwij,ocij->ohw", win, w, optimize=True)
    if b is not None:
        y = y + np.asarray(b, np.float64)[:, None, None]
    return y


def group_norm(x: np.ndarray, gamma, beta, groups: int, eps: float = 1e-5) -> np.ndarray:
    """GroupNorm of x [C][H][W] (population variance per group), float64."""
    x = np.asarray(x, np.float64)
    c = x.shape[0]
    g = x.reshape(groups, -1)
    mean = g.mean(axis=1, keepdims=True)
    var = g.var(axis=1, keepdims=True)
    y = ((g - mean) / np.sqrt(var + eps)).reshape(x.shape)
    return y * np.asarray(gamma, np.float64).reshape(c, 1, 1) + np.asarray(
        beta, np.float64).reshape(c, 1, 1)


def relu(x):
    return np.maximum(x, 0.0)


def max_pool(x: np.ndarray, k: int = 3, stride: int = 2, pad: int = 1) -> np.ndarray:
    """Max pool of x [C][H][W] with -inf padding."""
    xp = np.pad(np.asarray(x, np.float64), ((0, 0), (pad, pad), (pad, pad)),
                constant_values=-np.inf)
    hout = (xp.shape[1] - k) // stride + 1
    wout = (xp.shape[2] - k) // stride + 1
    win = np.lib.stride_tricks.sliding_window_view(xp, (k, k), axis=(1, 2))
    return win[:, ::stride, ::stride][:, :hout, :wout].max(axis=(3, 4))


def spatial_softmax(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Keypoints [K][2] of feature maps x [C][H][W]: 1x1 conv (w [K][C][1][1], b [K]), softmax
    over the positions, expected (x, y) on the [-1, 1] grid."""
    c, h, wd = x.shape
    logits = conv2d(x, w, b=b).reshape(w.shape[0], h * wd)
    logits = logits - logits.max(axis=1, keepdims=True)
    att = np.exp(logits)
    att = att / att.sum(axis=1, keepdims=True)
    pos_x, pos_y = np.meshgrid(np.linspace(-1.0, 1.0, wd), np.linspace(-1.0, 1.0, h))
    grid = np.stack([pos_x.reshape(-1), pos_y.reshape(-1)], axis=1)  # [H*W][2]
    return att @ grid


def _gn_groups(channels: int) -> int:
    return channels // 16


def backbone(t: dict, x: np.ndarray) -> np.ndarray:
    """resnet18 trunk (GroupNorm) on one cropped image x [3][h][w]; returns [512][h/32][w/32]."""
    p = "backbone."
    y = conv2d(x, t[p + "0.weight"], stride=2, pad=3)
    y = max_pool(relu(group_norm(y, t[p + "1.weight"], t[p + "1.bias"], _gn_groups(64))))
    cin = 64
    for s, cout in enumerate(STAGES):
        for blk in range(BLOCKS):
            q = f"{p}{4 + s}.{blk}."
            stride = 2 if (s > 0 and blk == 0) else 1
            h = conv2d(y, t[q + "conv1.weight"], stride=stride, pad=1)
            h = relu(group_norm(h, t[q + "bn1.weight"], t[q + "bn1.bias"], _gn_groups(cout)))
            h = conv2d(h, t[q + "conv2.weight"], stride=1, pad=1)
            h = group_norm(h, t[q + "bn2.weight"], t[q + "bn2.bias"], _gn_groups(cout))
            if q + "downsample.0.weight" in t:
                ident = conv2d(y, t[q + "downsample.0.weight"], stride=stride)
                ident = group_norm(ident, t[q + "downsample.1.weight"],
                                   t[q + "downsample.1.bias"], _gn_groups(cout))
            else:
                ident = y
            y = relu(h + ident)
        cin = cout
    return y


def encode(t: dict, image: np.ndarray, crop: tuple[int, int] | None) -> np.ndarray:
    """Feature vector [2 num_kp] of one image [3][H][W] (already normalized)."""
    x = np.asarray(image, np.float64)
    if crop is not None:
        top, left = center_crop_box(x.shape[1], x.shape[2], crop[0], crop[1])
        x = x[:, top:top + crop[0], left:left + crop[1]]
    kp = spatial_softmax(backbone(t, x), t["pool.nets.weight"], t["pool.nets.bias"])
    f = kp.reshape(-1)
    return relu(np.asarray(t["out.weight"], np.float64) @ f + np.asarray(t["out.bias"], np.float64))


def condition(states: np.ndarray, features: np.ndarray,
              env_states: np.ndarray | None = None) -> np.ndarray:
    """The head's condition: per observation step [state, image features (, env state)],
    flattened in step order (``observation.py:193-216``)."""
    parts = [np.asarray(states, np.float64), np.asarray(features, np.float64)]
    if env_states is not None:
        parts.append(np.asarray(env_states, np.float64))
    return np.concatenate(parts, axis=-1).reshape(-1)
