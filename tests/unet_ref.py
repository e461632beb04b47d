"""Test-side helpers: checkpoint builders and an independent float64 U-Net built on torch ops.

``torch_unet_eps`` composes ``torch.nn.functional.conv1d / conv_transpose1d / group_norm / mish``
in float64 following LeRobot's ``ConditionalUnet1d`` forward (down: two residual blocks, push
skip, downsample except on the last stage; two mid blocks; up: concat ``[x; skip]``, two
residual blocks, ConvTranspose upsample; final Conv1dBlock + 1x1 conv), with the FiLM
``scale * h + bias`` of each residual block.  It shares no code with the oracle.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from flowedge_amd import checkpoint as ck


def seq(count: int, frequency: float, phase: float) -> np.ndarray:
    """``sin(float(i) * frequency + phase)`` in float32, the reference test-fixture sequence."""
    i = np.arange(count, dtype=np.float32)
    return np.sin(i * np.float32(frequency) + np.float32(phase)).astype(np.float32)


def fixture_tensors():
    """The reference's 2-stage DiffusionFixture (``test/core_model_tests.cc:170-270``):
    dims (8, 16), H=4, A=2, cond=3, tdim=4, K=3, groups=2, T=10, sin-sequence weights."""
    out = []

    def add(name, arr):
        out.append((name, np.asarray(arr, dtype=np.float32)))

    def weights(count, phase):
        return seq(count, 0.173, phase) * np.float32(0.075)

    def conv(p, oc, ic, k, phase):
        add(p + ".w", weights(oc * ic * k, phase).reshape(oc, ic, k))
        add(p + ".b", np.full(oc, phase * 0.01, np.float32))

    def linear(p, o, i, phase):
        add(p + ".w", weights(o * i, phase).reshape(o, i))
        add(p + ".b", np.full(o, phase * 0.01, np.float32))

    def norm(p, c):
        add(p + ".w", np.ones(c, np.float32))
        add(p + ".b", np.zeros(c, np.float32))

    def residual(p, ic, oc, phase):
        conv(p + ".c1", oc, ic, 3, phase)
        norm(p + ".n1", oc)
        linear(p + ".film", 2 * oc, 4 + 3, phase + 0.01)
        conv(p + ".c2", oc, oc, 3, phase + 0.02)
        norm(p + ".n2", oc)
        if ic != oc:
            conv(p + ".res", oc, ic, 1, phase + 0.03)

    add("dp.meta", [1, 2, 4, 2, 2, 3, 2, 3, 2, 4, 10, 0, 0, 1, 1, 0])
    add("dp.dims", [8, 16])
    add("dp.action_min", [-2, 0])
    add("dp.action_max", [2, 10])
    linear("dp.te1", 16, 4, 0.01)
    linear("dp.te2", 4, 16, 0.02)
    residual("dp.d0.r0", 2, 8, 0.03)
    residual("dp.d0.r1", 8, 8, 0.04)
    conv("dp.d0.ds", 8, 8, 3, 0.05)
    residual("dp.d1.r0", 8, 16, 0.06)
    residual("dp.d1.r1", 16, 16, 0.07)
    residual("dp.m0", 16, 16, 0.08)
    residual("dp.m1", 16, 16, 0.09)
    residual("dp.u0.r0", 32, 8, 0.10)
    residual("dp.u0.r1", 8, 8, 0.11)
    conv("dp.u0.us", 8, 8, 4, 0.12)
    conv("dp.f.c", 8, 8, 3, 0.13)
    norm("dp.f.n", 8)
    conv("dp.f.o", 2, 8, 1, 0.14)
    return out


def write_fixture(path: str) -> str:
    ck.write_safetensors(path, fixture_tensors())
    return path


def write_variant(path: str, spec: ck.UNetSpec, seed: int = 0, zero=(), scale=None) -> str:
    """Synthetic checkpoint with the named tensors zeroed (e.g. ``dp.f.o.w``)."""
    tensors = []
    for name, arr in ck.synthetic_tensors(spec, seed):
        if name in zero:
            arr = np.zeros_like(arr)
        if scale and name in scale:
            arr = (arr * np.float32(scale[name])).astype(arr.dtype)
        tensors.append((name, arr))
    ck.write_safetensors(path, tensors)
    return path


def _t(a) -> torch.Tensor:
    a = np.asarray(a)
    if a.dtype == np.uint16:
        a = ck.bf16_widen(a)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64))


def torch_unet_eps(tensors: dict, cond, sample, t: float) -> np.ndarray:
    """Float64 ConditionalUnet1D forward; ``sample`` is ``[H][A]``; returns ``[H][A]``."""
    W = {k: _t(v) for k, v in tensors.items()}
    meta = [float(x) for x in tensors["dp.meta"]]
    A, H, stages, K, G, tdim = int(meta[1]), int(meta[2]), int(meta[6]), int(meta[7]), int(
        meta[8]), int(meta[9])
    dims = [int(d) for d in tensors["dp.dims"]]
    half = tdim // 2
    factor = math.log(10000.0) / (half - 1)
    freqs = torch.exp(-factor * torch.arange(half, dtype=torch.float64))
    ang = float(t) * freqs
    temb = torch.cat([torch.sin(ang), torch.cos(ang)])
    h = F.linear(temb, W["dp.te1.w"], W["dp.te1.b"])
    h = F.mish(h)
    temb = F.linear(h, W["dp.te2.w"], W["dp.te2.b"])
    gf = torch.cat([temb, _t(cond).reshape(-1)])

    def conv(x, p, stride=1, pad=None):
        w = W[p + ".w"]
        k = w.shape[2]
        return F.conv1d(x, w, W[p + ".b"], stride=stride, padding=k // 2 if pad is None else pad)

    def residual(x, p):
        oc = W[p + ".c1.w"].shape[0]
        out = F.mish(F.group_norm(conv(x, p + ".c1"), G, W[p + ".n1.w"], W[p + ".n1.b"]))
        emb = F.linear(F.mish(gf), W[p + ".film.w"], W[p + ".film.b"])
        out = emb[:oc].reshape(1, oc, 1) * out + emb[oc:].reshape(1, oc, 1)
        out = F.mish(F.group_norm(conv(out, p + ".c2"), G, W[p + ".n2.w"], W[p + ".n2.b"]))
        res = x if (p + ".res.w") not in W else conv(x, p + ".res")
        return out + res

    x = _t(sample).reshape(H, A).T.reshape(1, A, H)
    skips = []
    for s in range(stages):
        x = residual(x, f"dp.d{s}.r0")
        x = residual(x, f"dp.d{s}.r1")
        skips.append(x)
        if s + 1 < stages:
            x = conv(x, f"dp.d{s}.ds", stride=2, pad=1)
    x = residual(x, "dp.m0")
    x = residual(x, "dp.m1")
    for s in range(stages - 1):
        x = torch.cat([x, skips.pop()], dim=1)
        x = residual(x, f"dp.u{s}.r0")
        x = residual(x, f"dp.u{s}.r1")
        x = F.conv_transpose1d(x, W[f"dp.u{s}.us.w"], W[f"dp.u{s}.us.b"], stride=2, padding=1)
    x = F.mish(F.group_norm(conv(x, "dp.f.c"), 8, W["dp.f.n.w"], W["dp.f.n.b"]))
    x = conv(x, "dp.f.o")
    return x.reshape(A, H).T.numpy()


def alphas_cumprod_f64(T: int) -> np.ndarray:
    """squaredcos_cap_v2 in float64: prod(1 - min(1 - abar((i+1)/T)/abar(i/T), 0.999))."""
    def abar(x):
        return math.cos((x + 0.008) / 1.008 * math.pi / 2) ** 2
    out, c = [], 1.0
    for i in range(T):
        beta = min(1.0 - abar((i + 1) / T) / abar(i / T), 0.999)
        c *= 1.0 - beta
        out.append(c)
    return np.array(out)


def ddim_const_eps(noise, eps_const, steps: int, T: int, clip: float | None, amin, amax):
    """DDIM with an epsilon that is the same at every step, in float64."""
    ac = alphas_cumprod_f64(T)
    x = np.asarray(noise, np.float64).copy()
    e = np.asarray(eps_const, np.float64)
    ratio = T // steps
    for i in range(steps):
        ts = (steps - 1 - i) * ratio
        prev = ts - ratio
        at = ac[ts]
        ap = ac[prev] if prev >= 0 else 1.0
        x0 = (x - math.sqrt(1 - at) * e) / math.sqrt(at)
        if clip is not None:
            x0 = np.clip(x0, -clip, clip)
        x = math.sqrt(ap) * x0 + math.sqrt(1 - ap) * e
    return (x + 1) * 0.5 * (np.asarray(amax) - np.asarray(amin)) + np.asarray(amin)


def ddpm_const_eps(noise, eps_const, steps: int, T: int, clip: float | None, amin, amax,
                   seed: int):
    """DDPM posterior sampling (diffusers DDPMScheduler.step without variance clipping) with an
    epsilon that is the same at every step, in float64.

    x_prev = c0 clip(x0) + c1 x + sigma z with abar_t, abar_p = abar at t and t - T/steps (1 once
    negative), alpha = abar_t / abar_p, beta = 1 - alpha:
        c0 = sqrt(abar_p) beta / (1 - abar_t),  c1 = sqrt(alpha) (1 - abar_p) / (1 - abar_t),
        sigma^2 = (1 - abar_p) / (1 - abar_t) beta.
    z is the seeded Gaussian stream; it advances only on steps that add noise (every step but
    the last), one value per state entry in [t][a] order.
    """
    ac = alphas_cumprod_f64(T)
    x = np.asarray(noise, np.float64).copy()
    e = np.asarray(eps_const, np.float64)
    ratio = T // steps
    z = ck.gaussian(seed, max(steps - 1, 1) * x.size).astype(np.float64)
    drawn = 0
    for i in range(steps):
        ts = (steps - 1 - i) * ratio
        prev = ts - ratio
        at = ac[ts]
        ap = ac[prev] if prev >= 0 else 1.0
        x0 = (x - math.sqrt(1 - at) * e) / math.sqrt(at)
        if clip is not None:
            x0 = np.clip(x0, -clip, clip)
        alpha = at / ap
        beta = 1.0 - alpha
        nxt = math.sqrt(ap) * beta / (1 - at) * x0 + math.sqrt(alpha) * (1 - ap) / (1 - at) * x
        if prev >= 0:
            sigma = math.sqrt((1 - ap) / (1 - at) * beta)
            nxt = nxt + sigma * z[drawn:drawn + x.size].reshape(x.shape)
            drawn += x.size
        x = nxt
    return (x + 1) * 0.5 * (np.asarray(amax) - np.asarray(amin)) + np.asarray(amin)


# Shapes the checkpoint format admits beyond the common U-Net configurations: odd kernel sizes
# other than 3 and 5 (including 1), horizons that are not powers of two, more than 32 groups,
# widths that are not multiples of 16, width * length above 8192, more than 64 action dims and a
# final width above 1024.  Each keeps to the reference's validation (diffusion.cc:391-427).
GENERAL_SPECS = {
    "k7_h6_g3": ck.UNetSpec(dims=(24, 48), horizon=6, action_dim=3, cond_dim=5, kernel=7,
                            groups=3, timestep_dim=8, train_timesteps=50, action_steps=4,
                            obs_steps=2),
    "h12_stages3": ck.UNetSpec(dims=(32, 64, 96), horizon=12, action_dim=4, cond_dim=6,
                               kernel=5, groups=8, timestep_dim=16, action_steps=6),
    "h64_wide": ck.UNetSpec(dims=(256, 512), horizon=64, action_dim=2, cond_dim=20, kernel=5,
                            groups=8, timestep_dim=32, action_steps=8),
    "g64_k3": ck.UNetSpec(dims=(128, 256), horizon=16, action_dim=5, cond_dim=8, kernel=3,
                          groups=64, timestep_dim=16),
    "a70": ck.UNetSpec(dims=(32, 64), horizon=8, action_dim=70, cond_dim=6, kernel=5, groups=8,
                       timestep_dim=16, action_steps=4),
    "k1_c1088": ck.UNetSpec(dims=(1088, 1088), horizon=4, action_dim=6, cond_dim=10, kernel=1,
                            groups=8, timestep_dim=16, action_steps=2),
}
