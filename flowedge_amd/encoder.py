"""Observation encoder on the GPU: camera images and state to the Diffusion Policy condition.

``RgbEncoder`` wraps the library's ``fe_encoder_*`` C ABI (LeRobot's DiffusionRgbEncoder: center
crop, resnet18 trunk with GroupNorm, spatial-softmax keypoints, linear + ReLU, run as HIP
kernels).  ``DiffusionObservationEncoder`` is the counterpart of the reference's
``flowedge_lerobot.observation.DiffusionObservationEncoder``
(``integrations/lerobot/src/flowedge_lerobot/observation.py:152-216``): it keeps the last
``n_obs_steps`` observations (padding with the first one), and ``condition()`` returns, per step,
``[state, image features of every camera, environment state]``, flattened in step order, the
host vector ``Engine.sample_diffusion`` takes.  Without LeRobot in the environment the feature
names, shapes and normalization statistics are passed in explicitly (the reference reads them
from the source checkpoint's ``config.json`` and processor files).
"""

from __future__ import annotations

import ctypes
from collections import deque

import numpy as np

from . import checkpoint as _ck
from . import lib

_sz = ctypes.c_size_t
_fp = ctypes.POINTER(ctypes.c_float)


def _error() -> str:
    msg = lib().fe_engine_last_error()
    return msg.decode() if msg else ""


class RgbEncoder:
    """The Diffusion Policy RGB encoder on the GPU (one device arena, one graph per image count).

    ``path``: a safetensors file holding the encoder tensors under ``prefix`` (LeRobot's state
    dict names; ``diffusion.rgb_encoder.`` in a LeRobot ``model.safetensors``).
    """

    def __init__(self, path: str, prefix: str = _ck.ENCODER_PREFIX, image_hw=(96, 96),
                 crop_hw=(84, 84), max_images: int = 8):
        L = lib()
        ch, cw = crop_hw if crop_hw is not None else (0, 0)
        self._h = L.fe_encoder_load(path.encode(), prefix.encode(), image_hw[0], image_hw[1], ch,
                                    cw, max_images)
        if not self._h:
            raise RuntimeError(_error())
        c, f, k = _sz(), _sz(), _sz()
        self._check(L.fe_encoder_shape(self._h, ctypes.byref(c), ctypes.byref(f),
                                       ctypes.byref(k)))
        self.channels, self.feature_dim, self.keypoints = c.value, f.value, k.value
        self.image_hw = tuple(image_hw)
        self.max_images = max_images

    def _check(self, rc: int) -> None:
        if rc != 0:
            raise RuntimeError(_error())

    def encode(self, images) -> np.ndarray:
        """Features [n][F] of normalized images [n][C][H][W]."""
        x = np.ascontiguousarray(images, dtype=np.float32)
        if x.ndim != 4 or x.shape[1:] != (self.channels, *self.image_hw):
            raise ValueError(f"images must have shape [n, {self.channels}, {self.image_hw[0]}, "
                             f"{self.image_hw[1]}]")
        n = x.shape[0]
        out = np.empty((n, self.feature_dim), np.float32)
        self._check(lib().fe_encoder_encode(self._h, x.ctypes.data_as(_fp), n,
                                              out.ctypes.data_as(_fp)))
        return out

    def __call__(self, images) -> np.ndarray:
        return self.encode(images)

    def encode_device(self, images_ptr: int, n: int, out_ptr: int, out_stride: int,
                      out_offset: int = 0) -> None:
        """Device pointers: image i's features to out + i * out_stride + out_offset (floats)."""
        self._check(lib().fe_encoder_encode_device(self._h, images_ptr, n, out_ptr, out_stride,
                                                     out_offset))

    @property
    def last_device_ms(self) -> float:
        return float(lib().fe_encoder_last_device_ms(self._h))

    @property
    def device_bytes(self) -> int:
        return int(lib().fe_encoder_device_bytes(self._h))

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().fe_encoder_free(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()


def normalize(value, stats: dict | None, mode: str | None) -> np.ndarray:
    """LeRobot's input normalization: "mean_std" (x - mean) / (std + 1e-8), "min_max" to
    [-1, 1] by (x - min) / (max - min + 1e-8) * 2 - 1, or identity."""
    x = np.asarray(value, dtype=np.float32)
    if mode is None or stats is None:
        return x
    if mode == "mean_std":
        mean = np.asarray(stats["mean"], np.float32)
        std = np.asarray(stats["std"], np.float32)
        return (x - mean) / (std + np.float32(1e-8))
    if mode == "min_max":
        lo = np.asarray(stats["min"], np.float32)
        hi = np.asarray(stats["max"], np.float32)
        return (x - lo) / (hi - lo + np.float32(1e-8)) * np.float32(2) - np.float32(1)
    raise ValueError(f"unknown normalization mode {mode!r}")


class DiffusionObservationEncoder:
    """Observation history and condition assembly over an image encoder.

    ``encoder``: an ``RgbEncoder`` (or any callable mapping images [n][C][H][W] to features
    [n][F]).  ``input_features``: ``{name: shape}`` of the per-step inputs (without the batch
    dimension), in the source policy's order; ``state_key`` / ``image_keys`` /
    ``env_state_key`` name the state, camera and environment-state entries.  ``normalization``:
    ``{name: (mode, stats)}`` applied by ``observe`` unless ``normalized=True``.
    """

    def __init__(self, encoder, n_obs_steps: int, input_features: dict,
                 state_key: str = "observation.state", image_keys=("observation.image",),
                 env_state_key: str | None = None, normalization: dict | None = None):
        if n_obs_steps < 1:
            raise ValueError("n_obs_steps must be positive")
        if not image_keys:
            raise ValueError("visual adapter requires source image features")
        self.encoder = encoder
        self.n_obs_steps = n_obs_steps
        self.input_features = {k: tuple(v) for k, v in input_features.items()}
        self.state_key = state_key
        self.image_keys = tuple(image_keys)
        self.env_state_key = env_state_key
        self.normalization = dict(normalization or {})
        self.history: deque = deque(maxlen=n_obs_steps)

    def reset(self) -> None:
        self.history.clear()

    def observe(self, batch: dict, *, normalized: bool = False) -> None:
        """Record one observation step ({name: array of shape (1, *shape)})."""
        frame = {}
        for name, shape in self.input_features.items():
            value = batch.get(name)
            if value is None or tuple(np.shape(value)) != (1, *shape):
                raise ValueError(f"{name} must have shape {(1, *shape)} after preprocessing")
            v = np.asarray(value, dtype=np.float32)
            if not normalized and name in self.normalization:
                mode, stats = self.normalization[name]
                v = normalize(v, stats, mode)
            if not np.isfinite(v).all():
                raise ValueError(f"{name} contains non-finite values")
            frame[name] = np.array(v, dtype=np.float32, copy=True)
        if not self.history:
            self.history.extend([frame] * self.n_obs_steps)
        else:
            self.history.append(frame)

    def condition(self) -> np.ndarray:
        """The condition vector: per observation step [state, image features, env state]."""
        if not self.history:
            raise ValueError("observe must precede condition")
        n = self.n_obs_steps
        states = np.stack([f[self.state_key][0] for f in self.history])          # [n][S]
        images = np.stack([np.stack([f[k][0] for k in self.image_keys]) for f in self.history])
        features = np.asarray(self.encoder(images.reshape(-1, *images.shape[2:])),
                              np.float32).reshape(n, -1)                         # [n][cams * F]
        parts = [states, features]
        if self.env_state_key is not None:
            parts.append(np.stack([f[self.env_state_key][0] for f in self.history]))
        return np.ascontiguousarray(np.concatenate(parts, axis=-1).reshape(-1), np.float32)
