"""LeRobot Diffusion Policy deployment adapter over this library's Engine.

Same interface as FlowEdge's LeRobot adapter (integrations/lerobot/src/flowedge_lerobot/
diffusion.py:16-243, device check device.py:8-24): the caller keeps LeRobot's observation
encoder and feature normalisation and hands over the flattened condition vector and the initial
noise; the adapter validates them, runs one sampling call on the GPU and returns the part of the
predicted horizon that LeRobot executes.  LeRobot's diffusion policy predicts `horizon` actions
starting `observation_steps - 1` steps in the past and executes `action_steps` of them, i.e.
horizon rows [observation_steps - 1, observation_steps - 1 + action_steps).

LeRobot itself is not a dependency: the adapter only needs an engine with `diffusion_metadata`
and `sample_diffusion` (and uses `sample_diffusion_into` when present, to write the horizon into
storage it owns without a temporary).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Mapping, Protocol

import numpy as np

_CONTRACT_KEYS = ("condition_dim", "action_dim", "horizon", "action_steps", "observation_steps")
_SCHEDULERS = ("ddim", "ddpm")


class DiffusionEngine(Protocol):
    """What the adapter calls on an engine (flowedge_amd.Engine provides it)."""

    @property
    def diffusion_metadata(self) -> Mapping[str, Any]: ...

    def sample_diffusion(self, condition: np.ndarray, noise: np.ndarray, steps: int,
                         scheduler: str, seed: int) -> np.ndarray: ...


@dataclass(frozen=True)
class DiffusionActionContract:
    """The fixed shapes a converted checkpoint shares with LeRobot (diffusion.py:33-78)."""

    condition_dim: int
    action_dim: int
    horizon: int
    action_steps: int
    observation_steps: int

    @property
    def action_start(self) -> int:
        """Horizon row of the first action LeRobot executes (the current observation step)."""
        return self.observation_steps - 1

    @property
    def action_stop(self) -> int:
        return self.action_start + self.action_steps

    @classmethod
    def from_metadata(cls, metadata: Mapping[str, Any]) -> "DiffusionActionContract":
        """Contract from an engine's diffusion metadata; ValueError when it is incomplete or the
        executed slice does not fit in the horizon."""
        absent = [k for k in _CONTRACT_KEYS if k not in metadata]
        if absent:
            raise ValueError("missing diffusion metadata: " + ", ".join(absent))
        c = cls(**{k: int(metadata[k]) for k in _CONTRACT_KEYS})
        if min(c.condition_dim, c.action_dim, c.horizon, c.action_steps) <= 0:
            raise ValueError("diffusion dimensions must be positive")
        if c.observation_steps <= 0:
            raise ValueError("observation_steps must be positive")
        if c.action_stop > c.horizon:
            raise ValueError("LeRobot action slice is outside the diffusion horizon")
        return c


def require_device(device: str | None, engine: Any = None) -> None:
    """Fail-closed device check (device.py:8-24).  This library runs on the GPU only: "cuda" and
    "cuda:0" name the engine's device (the current HIP device at load, chosen with
    HIP_VISIBLE_DEVICES); "cpu" has no kernels here and is refused rather than emulated."""
    name = "cuda" if device is None else str(device)
    if name == "cpu":
        raise RuntimeError("this FlowEdge build has no CPU kernels; use device='cuda' on a "
                           "gfx950 GPU")
    if name not in ("cuda", "cuda:0"):
        raise ValueError("device must be 'cuda' or 'cuda:0' (select the GPU with "
                         "HIP_VISIBLE_DEVICES)")
    if engine is not None and not getattr(engine, "cuda_resident", False):
        raise RuntimeError("the engine is not device-resident")


class FlowEdgeDiffusionPolicy:
    """Deployment adapter for one converted LeRobot Diffusion Policy checkpoint
    (diffusion.py:80-243).  Returned actions are in dataset units (the engine unnormalises them);
    robot safety limits stay with the caller.  Not re-entrant, like the engine it wraps."""

    def __init__(self, engine: DiffusionEngine):
        self._engine = engine
        self.contract = DiffusionActionContract.from_metadata(engine.diffusion_metadata)
        c = self.contract
        self._horizon = np.empty((c.horizon, c.action_dim), np.float32)
        self._into = getattr(engine, "sample_diffusion_into", None)

    @classmethod
    def from_checkpoint(cls, path: str, *, threads: int | None = None,
                        device: str = "cuda") -> "FlowEdgeDiffusionPolicy":
        """Load a converted checkpoint onto the GPU."""
        from . import Engine

        require_device(device)
        engine = Engine(path, threads=threads)
        try:
            require_device(device, engine)
        except Exception:
            engine.close()
            raise
        return cls(engine)

    @property
    def engine(self) -> DiffusionEngine:
        return self._engine

    @property
    def metadata(self) -> DiffusionActionContract:
        return self.contract

    @property
    def cuda_resident(self) -> bool:
        return bool(getattr(self._engine, "cuda_resident", False))

    @property
    def action_dim(self) -> int:
        return self.contract.action_dim

    @property
    def action_steps(self) -> int:
        return self.contract.action_steps

    def reset(self) -> None:
        """Nothing to reset: every sampling call is independent of the previous ones."""

    def predict_action_chunk(self, condition, noise, *, steps: int = 10,
                             scheduler: str = "ddim", seed: int = 0) -> np.ndarray:
        """The executed action chunk [action_steps][action_dim] for one condition."""
        out = np.empty((self.contract.action_steps, self.contract.action_dim), np.float32)
        return self.predict_action_chunk_into(condition, noise, out, steps=steps,
                                              scheduler=scheduler, seed=seed)

    def predict_action_chunk_into(self, condition, noise, output: np.ndarray, *,
                                  steps: int = 10, scheduler: str = "ddim",
                                  seed: int = 0) -> np.ndarray:
        """Writes the executed action chunk into caller-owned float32 storage and returns it."""
        c = self.contract
        _check_output(output, (c.action_steps, c.action_dim))
        self._sample(condition, noise, steps, scheduler, seed)
        output[...] = self._horizon[c.action_start:c.action_stop]
        return output

    def select_action(self, condition, noise, *, steps: int = 10, scheduler: str = "ddim",
                      seed: int = 0) -> np.ndarray:
        """The first executed action, for loops that act one step per observation."""
        out = np.empty(self.contract.action_dim, np.float32)
        return self.select_action_into(condition, noise, out, steps=steps, scheduler=scheduler,
                                       seed=seed)

    def select_action_into(self, condition, noise, output: np.ndarray, *, steps: int = 10,
                           scheduler: str = "ddim", seed: int = 0) -> np.ndarray:
        _check_output(output, (self.contract.action_dim,))
        self._sample(condition, noise, steps, scheduler, seed)
        output[...] = self._horizon[self.contract.action_start]
        return output

    def _sample(self, condition, noise, steps: int, scheduler: str, seed: int) -> None:
        """One sampling call into self._horizon, after the argument checks of diffusion.py:205-225
        (ValueError, before the engine is called)."""
        c = self.contract
        cond = np.ascontiguousarray(condition, dtype=np.float32).reshape(-1)
        x = np.ascontiguousarray(noise, dtype=np.float32)
        if cond.size != c.condition_dim:
            raise ValueError(f"condition must contain {c.condition_dim} float32 values")
        if x.shape != self._horizon.shape:
            raise ValueError(f"noise must have shape {self._horizon.shape}")
        if steps <= 0:
            raise ValueError("steps must be positive")
        if scheduler not in _SCHEDULERS:
            raise ValueError("scheduler must be one of: " + ", ".join(_SCHEDULERS))
        if self._into is not None:
            self._into(cond, x, self._horizon, steps, scheduler, int(seed))
            return
        got = np.asarray(self._engine.sample_diffusion(cond, x, steps, scheduler, int(seed)),
                         dtype=np.float32)
        if got.shape != self._horizon.shape:
            raise ValueError(f"engine returned a horizon of shape {got.shape}, expected "
                             f"{self._horizon.shape}")
        self._horizon[...] = got


def _check_output(output, shape: tuple[int, ...]) -> None:
    if not (isinstance(output, np.ndarray) and output.shape == shape and
            output.dtype == np.float32 and output.flags["C_CONTIGUOUS"]):
        raise ValueError(f"output must be a C-contiguous float32 array of shape {shape}")
