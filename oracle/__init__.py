"""ctypes wrapper of the CPU oracle (``dp_oracle.cpp``) — test infrastructure only.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``, always as the checker (or the timed CPU baseline), never as the measured GPU path.

Parity pins for each oracle function (the tests that fix it):
  conv1d / 1x1 / stride-2 ... brute-force cross-correlation and torch.nn.functional.conv1d
  conv_transpose1d .......... naive scatter and torch.nn.functional.conv_transpose1d
  group_norm ................ closed form in float64 and torch.nn.functional.group_norm
  mish ...................... libm x*tanh(log1p(e^x)), torch mish, saturation at +-30
  timestep embedding ........ closed form at t = 0 (sin 0 / cos 1) and a float64 restatement
  matmul .................... float64 product
  alphas_cumprod ............ squaredcos closed form (float64) and monotonicity
  Gaussian .................. splitmix64 vectors (published first outputs) and Box-Muller identity
  denoise ................... composition of the pinned ops (float64 numpy U-Net restatement on
                              the tiny model), zeroed output conv => eps == bias, determinism and
                              conditioning sensitivity
  DDIM / DDPM ............... closed-form update on a mocked eps, clip invariant (actions inside
                              [min, max]), seed independence (DDIM) and seed dependence (DDPM)
  flow ODE .................. Euler/RK4 on a zeroed velocity network (constant v = bias)
  partial samples ........... closed form after k of n steps on a constant epsilon / velocity
                              (fixes the timestep of each step); k = n equals the whole sample
  model fingerprint ......... fingerprint.py: XXH64 from the independent xxhash package; the
                              composition is restated and checked by its sensitivity invariants
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_dp.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u64p = ctypes.POINTER(ctypes.c_uint64)


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (g++)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.dpo_last_error.restype = ctypes.c_char_p
        L.dpo_load.restype = ctypes.c_void_p
        L.dpo_load.argtypes = [ctypes.c_char_p, ctypes.c_uint]
        L.dpo_free.argtypes = [ctypes.c_void_p]
        L.dpo_config.argtypes = [ctypes.c_void_p, _u64p, _u64p, _f32p]
        L.dpo_alphas_cumprod.argtypes = [ctypes.c_void_p, _f32p]
        L.dpo_denoise.argtypes = [ctypes.c_void_p, _f32p, _f32p, ctypes.c_float, _f32p]
        L.dpo_sample.argtypes = [ctypes.c_void_p, _f32p, _f32p, ctypes.c_size_t, ctypes.c_int,
                                 ctypes.c_uint64, _f32p]
        L.dpo_sample_flow.argtypes = [ctypes.c_void_p, _f32p, _f32p, ctypes.c_size_t,
                                      ctypes.c_int, _f32p]
        L.dpo_sample_partial.argtypes = [ctypes.c_void_p, _f32p, _f32p, ctypes.c_size_t,
                                         ctypes.c_int, ctypes.c_uint64, ctypes.c_size_t, _f32p]
        L.dpo_sample_flow_partial.argtypes = [ctypes.c_void_p, _f32p, _f32p, ctypes.c_size_t,
                                              ctypes.c_int, ctypes.c_size_t, _f32p]
        L.dpo_sample_batch.argtypes = [ctypes.c_void_p, ctypes.c_size_t, _f32p, _f32p,
                                       ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_uint64, _f32p, ctypes.c_uint]
        L.dpo_mish.argtypes = [_f32p, ctypes.c_size_t]
        L.dpo_timestep_embedding.argtypes = [ctypes.c_float, _f32p, ctypes.c_size_t]
        L.dpo_matmul.argtypes = [_f32p, _f32p, _f32p] + [ctypes.c_size_t] * 3
        L.dpo_conv1d.argtypes = [_f32p] * 4 + [ctypes.c_size_t] * 7
        L.dpo_conv_transpose1d.argtypes = [_f32p] * 4 + [ctypes.c_size_t] * 7
        L.dpo_group_norm.argtypes = [_f32p] * 3 + [ctypes.c_size_t] * 3
        L.dpo_gaussian.argtypes = [ctypes.c_uint64, _f32p, ctypes.c_size_t]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    """One loaded checkpoint on the CPU oracle."""

    def __init__(self, path: str, threads: int = 0):
        self._h = lib().dpo_load(path.encode(), threads)
        if not self._h:
            raise RuntimeError("oracle load failed: " + lib().dpo_last_error().decode())
        v = (ctypes.c_uint64 * 12)()
        d = (ctypes.c_uint64 * 8)()
        cr = ctypes.c_float()
        lib().dpo_config(self._h, v, d, ctypes.byref(cr))
        (self.action_dim, self.horizon, self.cond_dim, self.stages, self.kernel, self.groups,
         self.timestep_dim, self.train_timesteps, clip, self.prediction, self.action_steps,
         self.obs_steps) = [int(x) for x in v]
        self.clip_sample = bool(clip)
        self.clip_range = cr.value
        self.dims = tuple(int(d[i]) for i in range(self.stages))

    def close(self):
        if getattr(self, "_h", None):
            lib().dpo_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may already be unloaded
            pass

    @property
    def values(self) -> int:
        return self.horizon * self.action_dim

    def alphas_cumprod(self) -> np.ndarray:
        out = np.empty(self.train_timesteps, np.float32)
        lib().dpo_alphas_cumprod(self._h, _p(out))
        return out

    def denoise(self, cond, sample, t: float) -> np.ndarray:
        cond, sample = _f(cond), _f(sample)
        out = np.empty(self.values, np.float32)
        rc = lib().dpo_denoise(self._h, _p(cond), _p(sample), float(t), _p(out))
        if rc:
            raise RuntimeError(f"oracle denoise failed ({rc})")
        return out.reshape(self.horizon, self.action_dim)

    def sample(self, cond, noise, steps: int, scheduler: int = 0, seed: int = 0) -> np.ndarray:
        cond, noise = _f(cond), _f(noise)
        out = np.empty(self.values, np.float32)
        rc = lib().dpo_sample(self._h, _p(cond), _p(noise), steps, scheduler, seed, _p(out))
        if rc:
            raise RuntimeError(f"oracle sample failed ({rc})")
        return out.reshape(self.horizon, self.action_dim)

    def sample_partial(self, cond, noise, steps: int, done: int, scheduler: int = 0,
                       seed: int = 0) -> np.ndarray:
        """The first `done` of `steps` DDIM/DDPM steps; the sample in action units."""
        cond, noise = _f(cond), _f(noise)
        out = np.empty(self.values, np.float32)
        rc = lib().dpo_sample_partial(self._h, _p(cond), _p(noise), steps, scheduler, seed, done,
                                      _p(out))
        if rc:
            raise RuntimeError(f"oracle partial sample failed ({rc})")
        return out.reshape(self.horizon, self.action_dim)

    def sample_flow_partial(self, cond, x0, steps: int, method: int, done: int) -> np.ndarray:
        """The first `done` of `steps` ODE steps."""
        cond, x0 = _f(cond), _f(x0)
        out = np.empty(self.values, np.float32)
        rc = lib().dpo_sample_flow_partial(self._h, _p(cond), _p(x0), steps, method, done,
                                           _p(out))
        if rc:
            raise RuntimeError(f"oracle partial flow sample failed ({rc})")
        return out.reshape(self.horizon, self.action_dim)

    def sample_flow(self, cond, x0, steps: int, method: int) -> np.ndarray:
        cond, x0 = _f(cond), _f(x0)
        out = np.empty(self.values, np.float32)
        rc = lib().dpo_sample_flow(self._h, _p(cond), _p(x0), steps, method, _p(out))
        if rc:
            raise RuntimeError(f"oracle flow sample failed ({rc})")
        return out.reshape(self.horizon, self.action_dim)

    def sample_batch(self, cond, noise, steps: int, kind: int = 0, mode: int = 0, seed: int = 0,
                     workers: int = 1) -> np.ndarray:
        cond, noise = _f(cond), _f(noise)
        b = cond.shape[0]
        out = np.empty((b, self.horizon, self.action_dim), np.float32)
        rc = lib().dpo_sample_batch(self._h, b, _p(cond), _p(noise), steps, kind, mode, seed,
                                    _p(out), workers)
        if rc:
            raise RuntimeError(f"oracle batch sample failed ({rc})")
        return out


# ---- op-level helpers (unit tests) ----
def mish(x) -> np.ndarray:
    x = _f(x).copy()
    lib().dpo_mish(_p(x), x.size)
    return x


def timestep_embedding(t: float, dim: int) -> np.ndarray:
    out = np.empty(dim, np.float32)
    lib().dpo_timestep_embedding(float(t), _p(out), dim)
    return out


def matmul(inp, w) -> np.ndarray:
    inp, w = _f(inp), _f(w)
    out = np.empty((inp.shape[0], w.shape[0]), np.float32)
    lib().dpo_matmul(_p(inp), _p(w), _p(out), inp.shape[0], inp.shape[1], w.shape[0])
    return out


def conv1d(x, w, b, stride: int = 1, pad: int | None = None) -> np.ndarray:
    x, w, b = _f(x), _f(w), _f(b)
    oc, ic, k = w.shape
    lin = x.shape[1]
    pad = k // 2 if pad is None else pad
    lout = (lin + 2 * pad - k) // stride + 1
    y = np.empty((oc, lout), np.float32)
    lib().dpo_conv1d(_p(x), _p(w), _p(b), _p(y), ic, oc, lin, lout, k, stride, pad)
    return y


def conv_transpose1d(x, w, b, stride: int = 2, pad: int = 1) -> np.ndarray:
    x, w, b = _f(x), _f(w), _f(b)
    ic, oc, k = w.shape
    lin = x.shape[1]
    lout = (lin - 1) * stride - 2 * pad + k
    y = np.empty((oc, lout), np.float32)
    lib().dpo_conv_transpose1d(_p(x), _p(w), _p(b), _p(y), ic, oc, lin, lout, k, stride, pad)
    return y


def group_norm(x, w, b, groups: int) -> np.ndarray:
    x, w, b = _f(x).copy(), _f(w), _f(b)
    c, length = x.shape
    lib().dpo_group_norm(_p(x), _p(w), _p(b), c, length, groups)
    return x


def gaussian(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().dpo_gaussian(seed, _p(out), n)
    return out
