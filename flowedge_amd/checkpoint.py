"""Diffusion Policy checkpoints in FlowEdge's ``dp.*`` safetensors layout.

The tensor names, shapes and the 16-float ``dp.meta`` record follow the reference converter
(``convert/convert.py:440-574``) and the loader contract (``src/core/heads/diffusion/
diffusion.cc:391-527``):

``dp.meta = [schema=1, action_dim, horizon, action_steps, obs_steps, cond_dim, stages, kernel,
groups, timestep_dim, train_timesteps, beta_schedule=0, prediction_type, clip_sample,
clip_sample_range, normalization=0]``

``prediction_type`` 0 is epsilon (the reference); 1 marks the U-Net as a flow-matching velocity
field (an extension of this library).  Conv and linear weights may be stored as BF16 (conv BF16 is
an extension; the reference accepts BF16 only for linears, which is the layout its converter
writes with ``--dtype bf16``: 2-D weights BF16, everything else F32, ``convert.py:602-610``).

Synthetic weights use PyTorch's default ``Conv1d``/``Linear`` initialisation bound
``U(-1/sqrt(fan_in), +1/sqrt(fan_in))`` for weight and bias (ConvTranspose takes ``fan_in`` from
dim 1 of its ``[IC][OC][K]`` storage), drawn from one splitmix64 stream seeded 0 in ``dp.*`` key
order; GroupNorm weight 1, bias 0; action range [-1, 1].  Conditions and initial noise come from
the reference's seeded Gaussian (splitmix64 + Box-Muller, ``diffusion.cc:193-231``).
"""

from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass, field

import numpy as np

GAMMA = 0x9E3779B97F4A7C15
_M1 = 0xBF58476D1CE4E5B9
_M2 = 0x94D049BB133111EB


@dataclass
class UNetSpec:
    """Shape of a ConditionalUnet1D action head."""

    dims: tuple = (512, 1024, 2048)
    action_dim: int = 2
    horizon: int = 16
    cond_dim: int = 132
    kernel: int = 5
    groups: int = 8
    timestep_dim: int = 128
    train_timesteps: int = 100
    action_steps: int = 8
    obs_steps: int = 2
    clip_sample: bool = True
    clip_range: float = 1.0
    prediction: int = 0  # 0 epsilon (DDIM/DDPM), 1 velocity (flow ODE)
    bf16_weights: bool = False  # every weight tensor BF16 (BF16 convolutions: an extension)
    bf16_linears: bool = False  # only 2-D linear weights BF16 (the converter's --dtype bf16)
    action_min: tuple | None = None
    action_max: tuple | None = None

    def meta(self) -> np.ndarray:
        return np.array(
            [1, self.action_dim, self.horizon, self.action_steps, self.obs_steps, self.cond_dim,
             len(self.dims), self.kernel, self.groups, self.timestep_dim, self.train_timesteps,
             0, self.prediction, int(bool(self.clip_sample)), self.clip_range, 0],
            dtype=np.float32)


# Named workloads.  "tiny" is the CPU-runnable plumbing case; "pusht" is the LeRobot-default
# (diffusion_pusht) size; "bimanual" the horizon-8 / 14-dof BF16 variant; "flow" the U-Net
# velocity-field head.
SPECS = {
    "tiny": UNetSpec(dims=(64, 128, 256), cond_dim=64),
    "pusht": UNetSpec(),
    "bimanual": UNetSpec(horizon=8, action_dim=14, cond_dim=1052, action_steps=4,
                         bf16_weights=True),
    "flow": UNetSpec(action_dim=7, cond_dim=256, prediction=1),
}


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(_M1)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(_M2)
    return z ^ (z >> np.uint64(31))


def splitmix_u64(seed: int, start: int, count: int) -> np.ndarray:
    """Raw outputs of calls ``start .. start+count-1`` of the reference's splitmix64 stream.

    The state starts at ``seed + GAMMA`` and each call adds GAMMA before mixing, so call ``i``
    mixes ``seed + (i + 2) * GAMMA`` (``diffusion.cc:196, 214-221``).
    """
    with np.errstate(over="ignore"):
        idx = np.arange(start + 2, start + 2 + count, dtype=np.uint64)
        return _mix(np.uint64(seed % (1 << 64)) + idx * np.uint64(GAMMA))


def splitmix_uniform(seed: int, start: int, count: int) -> np.ndarray:
    """Uniforms ``((z >> 40) + 1) / 16777217`` in float32 (``diffusion.cc:223-226``).

    Computed in chunks of 2^16 calls with reused buffers (large temporaries would each be mapped
    and faulted in afresh)."""
    out = np.empty(count, dtype=np.float32)
    chunk = 1 << 16
    base = np.arange(2, 2 + chunk, dtype=np.uint64)
    z = np.empty(chunk, dtype=np.uint64)
    t = np.empty(chunk, dtype=np.uint64)
    seed64 = np.uint64(seed % (1 << 64))
    with np.errstate(over="ignore"):
        for lo in range(0, count, chunk):
            n = min(chunk, count - lo)
            zz, tt = z[:n], t[:n]
            # state after call (start + lo + i): seed + (start + lo + i + 2) * GAMMA
            np.add(base[:n], np.uint64(start + lo), out=zz)
            np.multiply(zz, np.uint64(GAMMA), out=zz)
            np.add(zz, seed64, out=zz)
            np.right_shift(zz, np.uint64(30), out=tt)
            np.bitwise_xor(zz, tt, out=zz)
            np.multiply(zz, np.uint64(_M1), out=zz)
            np.right_shift(zz, np.uint64(27), out=tt)
            np.bitwise_xor(zz, tt, out=zz)
            np.multiply(zz, np.uint64(_M2), out=zz)
            np.right_shift(zz, np.uint64(31), out=tt)
            np.bitwise_xor(zz, tt, out=zz)
            np.right_shift(zz, np.uint64(40), out=zz)
            np.add(zz, np.uint64(1), out=zz)
            o = out[lo:lo + n]
            o[...] = zz
            np.divide(o, np.float32(16777217.0), out=o)
    return out


def gaussian(seed: int, count: int) -> np.ndarray:
    """``count`` values of the reference's seeded Gaussian stream (Box-Muller, cos first)."""
    pairs = (count + 1) // 2
    u = splitmix_uniform(seed, 0, 2 * pairs)
    first = np.maximum(u[0::2], np.finfo(np.float32).tiny)
    second = u[1::2]
    radius = np.sqrt(np.float32(-2.0) * np.log(first)).astype(np.float32)
    angle = (np.float32(2.0 * np.float32(np.pi)) * second).astype(np.float32)
    out = np.empty(2 * pairs, dtype=np.float32)
    out[0::2] = radius * np.cos(angle)
    out[1::2] = radius * np.sin(angle)
    return out[:count]


def bf16_round(values: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest BF16 (ties to even); returns the uint16 bit patterns."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    rounding = np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))
    return ((bits + rounding) >> np.uint32(16)).astype(np.uint16)


def bf16_widen(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def layout(spec: UNetSpec):
    """Yield ``(name, shape, kind, fan_in)`` in ``dp.*`` key order.

    ``kind``: "w" (random weight), "b" (random bias), "one"/"zero" (GroupNorm affine).
    Mirrors the converter's mapping order (``convert.py:498-573``).
    """
    dims, k, t, c = list(spec.dims), spec.kernel, spec.timestep_dim, spec.cond_dim
    film = t + c

    def conv(p, oc, ic, kk):
        yield p + ".w", (oc, ic, kk), "w", ic * kk
        yield p + ".b", (oc,), "b", ic * kk

    def convt(p, ch, kk):  # ConvTranspose1d storage [IC][OC][K]; fan_in = OC*K
        yield p + ".w", (ch, ch, kk), "w", ch * kk
        yield p + ".b", (ch,), "b", ch * kk

    def linear(p, out, inp):
        yield p + ".w", (out, inp), "w", inp
        yield p + ".b", (out,), "b", inp

    def norm(p, ch):
        yield p + ".w", (ch,), "one", 0
        yield p + ".b", (ch,), "zero", 0

    def residual(p, ic, oc):
        yield from conv(p + ".c1", oc, ic, k)
        yield from norm(p + ".n1", oc)
        yield from linear(p + ".film", 2 * oc, film)
        yield from conv(p + ".c2", oc, oc, k)
        yield from norm(p + ".n2", oc)
        if ic != oc:
            yield from conv(p + ".res", oc, ic, 1)

    yield from linear("dp.te1", 4 * t, t)
    yield from linear("dp.te2", t, 4 * t)
    for s, oc in enumerate(dims):
        ic = spec.action_dim if s == 0 else dims[s - 1]
        yield from residual(f"dp.d{s}.r0", ic, oc)
        yield from residual(f"dp.d{s}.r1", oc, oc)
        if s + 1 < len(dims):
            yield from conv(f"dp.d{s}.ds", oc, oc, 3)
    for b in range(2):
        yield from residual(f"dp.m{b}", dims[-1], dims[-1])
    for s in range(len(dims) - 1):
        high, low = dims[-1 - s], dims[-2 - s]
        yield from residual(f"dp.u{s}.r0", 2 * high, low)
        yield from residual(f"dp.u{s}.r1", low, low)
        yield from convt(f"dp.u{s}.us", low, 4)
    yield from conv("dp.f.c", dims[0], dims[0], k)
    yield from norm("dp.f.n", dims[0])
    yield from conv("dp.f.o", spec.action_dim, dims[0], 1)


def synthetic_tensors(spec: UNetSpec, seed: int = 0):
    """Yield ``(name, array)``; BF16 weights are uint16 bit patterns."""
    cursor = 0
    for name, shape, kind, fan_in in layout(spec):
        count = int(np.prod(shape))
        if kind in ("w", "b"):
            bound = np.float32(1.0 / np.sqrt(fan_in))
            values = splitmix_uniform(seed, cursor, count)
            cursor += count
            # (2u - 1) * bound, in place (each step rounds to float32 as the plain expression)
            np.multiply(values, np.float32(2.0), out=values)
            np.subtract(values, np.float32(1.0), out=values)
            np.multiply(values, bound, out=values)
            values = values.reshape(shape)
            if kind == "w" and (spec.bf16_weights or (spec.bf16_linears and len(shape) == 2)):
                values = bf16_round(values)
            yield name, values
        elif kind == "one":
            yield name, np.ones(shape, dtype=np.float32)
        else:
            yield name, np.zeros(shape, dtype=np.float32)
    amin = np.full(spec.action_dim, -1.0, np.float32) if spec.action_min is None else np.asarray(
        spec.action_min, np.float32)
    amax = np.full(spec.action_dim, 1.0, np.float32) if spec.action_max is None else np.asarray(
        spec.action_max, np.float32)
    yield "dp.action_min", amin
    yield "dp.action_max", amax
    yield "dp.dims", np.asarray(spec.dims, dtype=np.float32)
    yield "dp.meta", spec.meta()


def write_safetensors(path: str, tensors) -> int:
    """Write ``(name, array)`` pairs (float32, or uint16 = BF16 bits).  Returns bytes written."""
    items = [(n, np.ascontiguousarray(a)) for n, a in tensors]
    header, offset = {}, 0
    for name, arr in items:
        dtype = "BF16" if arr.dtype == np.uint16 else "F32"
        if dtype == "F32" and arr.dtype != np.float32:
            raise TypeError(f"{name}: unsupported dtype {arr.dtype}")
        header[name] = {"dtype": dtype, "shape": list(arr.shape),
                        "data_offsets": [offset, offset + arr.nbytes]}
        offset += arr.nbytes
    blob = json.dumps(header, separators=(",", ":")).encode()
    blob += b" " * ((8 - len(blob) % 8) % 8)
    tmp = f"{path}.tmp{os.getpid()}"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(blob)))
        f.write(blob)
        for _, arr in items:
            f.write(arr.tobytes())
    os.replace(tmp, path)
    return 8 + len(blob) + offset


def read_safetensors(path: str) -> dict:
    """Read a safetensors file into ``{name: array}`` (BF16 as uint16 bits); executes nothing."""
    out = {}
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(n))
        base = 8 + n
        for name, info in header.items():
            if name == "__metadata__":
                continue
            lo, hi = info["data_offsets"]
            f.seek(base + lo)
            raw = f.read(hi - lo)
            dt = {"F32": np.float32, "BF16": np.uint16}[info["dtype"]]
            out[name] = np.frombuffer(raw, dtype=dt).reshape(info["shape"]).copy()
    return out


def write_synthetic(path: str, spec: UNetSpec, seed: int = 0) -> str:
    write_safetensors(path, synthetic_tensors(spec, seed))
    return path


def cached_checkpoint(workload: str, directory: str | None = None, seed: int = 0) -> str:
    """Path of the synthetic checkpoint for a named workload, generating it once."""
    spec = SPECS[workload]
    directory = directory or os.environ.get("FLOWEDGE_CKPT_DIR") or os.path.join(
        os.environ.get("TMPDIR", "/tmp"), "flowedge_ckpt")
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, f"dp_{workload}_seed{seed}.safetensors")
    if not os.path.exists(path):
        write_synthetic(path, spec, seed)
    return path


def inputs(spec: UNetSpec, batch: int = 1, cond_seed: int = 1, noise_seed: int = 2):
    """Seeded condition ``[B, cond]`` and initial noise ``[B, H, A]`` (one stream each)."""
    cond = gaussian(cond_seed, batch * spec.cond_dim).reshape(batch, spec.cond_dim)
    noise = gaussian(noise_seed, batch * spec.horizon * spec.action_dim).reshape(
        batch, spec.horizon, spec.action_dim)
    return cond, noise


# ---- Observation encoder (LeRobot DiffusionRgbEncoder: resnet18 + GroupNorm + SpatialSoftmax) ----

ENCODER_PREFIX = "diffusion.rgb_encoder."


@dataclass
class EncoderSpec:
    """Shape of a Diffusion Policy RGB encoder: resnet18 widths, crop and keypoints."""

    channels: int = 3
    image_hw: tuple = (96, 96)   # camera image (pusht)
    crop_hw: tuple | None = (84, 84)
    keypoints: int = 32
    stages: tuple = (64, 128, 256, 512)

    def feature_map_hw(self) -> tuple:
        h, w = self.crop_hw if self.crop_hw is not None else self.image_hw
        for _ in range(5):  # stem conv, max pool, stages 2-4: stride 2 each, padding "same"
            h, w = (h + 1) // 2, (w + 1) // 2
        return h, w


def encoder_layout(spec: EncoderSpec):
    """Yield ``(name, shape, kind, fan_in)`` of the encoder's state dict (LeRobot names, without
    the ``diffusion.rgb_encoder.`` prefix).  ``kind``: "w" (weight), "b" (bias), "gw"/"gb"
    (GroupNorm affine), "grid" (SpatialSoftmax position buffer)."""
    c0 = spec.stages[0]
    yield "backbone.0.weight", (c0, spec.channels, 7, 7), "w", spec.channels * 49
    yield "backbone.1.weight", (c0,), "gw", 0
    yield "backbone.1.bias", (c0,), "gb", 0
    cin = c0
    for s, cout in enumerate(spec.stages):
        for blk in range(2):
            p = f"backbone.{4 + s}.{blk}."
            ic = cin if blk == 0 else cout
            yield p + "conv1.weight", (cout, ic, 3, 3), "w", ic * 9
            yield p + "bn1.weight", (cout,), "gw", 0
            yield p + "bn1.bias", (cout,), "gb", 0
            yield p + "conv2.weight", (cout, cout, 3, 3), "w", cout * 9
            yield p + "bn2.weight", (cout,), "gw", 0
            yield p + "bn2.bias", (cout,), "gb", 0
            if blk == 0 and s > 0:
                yield p + "downsample.0.weight", (cout, ic, 1, 1), "w", ic
                yield p + "downsample.1.weight", (cout,), "gw", 0
                yield p + "downsample.1.bias", (cout,), "gb", 0
        cin = cout
    k = spec.keypoints
    h, w = spec.feature_map_hw()
    yield "pool.nets.weight", (k, cin, 1, 1), "w", cin
    yield "pool.nets.bias", (k,), "b", cin
    yield "pool.pos_grid", (h * w, 2), "grid", 0
    yield "out.weight", (2 * k, 2 * k), "w", 2 * k
    yield "out.bias", (2 * k,), "b", 2 * k


def synthetic_encoder_tensors(spec: EncoderSpec, seed: int = 3, prefix: str = ENCODER_PREFIX):
    """Yield ``(name, float32 array)``: weights and biases U(+-1/sqrt(fan_in)) as PyTorch's
    default initialisation, GroupNorm affine 1 + U(+-0.1) and U(+-0.1) (so the affine terms are
    exercised), drawn from one splitmix64 stream in layout order."""
    cursor = 0
    for name, shape, kind, fan_in in encoder_layout(spec):
        count = int(np.prod(shape))
        if kind == "grid":
            h, w = spec.feature_map_hw()
            px, py = np.meshgrid(np.linspace(-1.0, 1.0, w), np.linspace(-1.0, 1.0, h))
            yield prefix + name, np.stack([px.reshape(-1), py.reshape(-1)], 1).astype(np.float32)
            continue
        u = splitmix_uniform(seed, cursor, count).astype(np.float64)
        cursor += count
        if kind in ("w", "b"):
            v = (2.0 * u - 1.0) / np.sqrt(fan_in)
        elif kind == "gw":
            v = 1.0 + 0.1 * (2.0 * u - 1.0)
        else:
            v = 0.1 * (2.0 * u - 1.0)
        yield prefix + name, v.astype(np.float32).reshape(shape)


def cached_encoder(directory: str | None = None, spec: EncoderSpec | None = None,
                   seed: int = 3) -> str:
    """Path of a synthetic encoder checkpoint (LeRobot tensor names), generated once."""
    spec = spec or EncoderSpec()
    directory = directory or os.environ.get("FLOWEDGE_CKPT_DIR") or os.path.join(
        os.environ.get("TMPDIR", "/tmp"), "flowedge_ckpt")
    os.makedirs(directory, exist_ok=True)
    tag = f"{spec.image_hw[0]}x{spec.image_hw[1]}_c{spec.channels}_k{spec.keypoints}"
    path = os.path.join(directory, f"rgb_encoder_{tag}_seed{seed}.safetensors")
    if not os.path.exists(path):
        write_safetensors(path, synthetic_encoder_tensors(spec, seed))
    return path


def encoder_images(spec: EncoderSpec, n: int, seed: int = 5) -> np.ndarray:
    """``n`` normalized images [n][C][H][W] from the seeded Gaussian stream."""
    h, w = spec.image_hw
    return gaussian(seed, n * spec.channels * h * w).reshape(n, spec.channels, h, w)
