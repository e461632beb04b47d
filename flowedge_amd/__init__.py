"""FlowEdge Diffusion Policy engine on AMD Instinct MI355X.

``Engine`` mirrors the reference's ``flowedge.Engine`` binding (``python/flowedge_ext.cc:518-561,
791-847``) for the Diffusion Policy path: same constructor, properties and method names, numpy in
and out, errors raised as ``RuntimeError`` with ``fe_engine_last_error()``.  Every call goes
through the C ABI in ``include/flowedge.h`` (``libflowedge_amd.so``); there is no host fallback:
if the library is not built, importing the binding fails.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import checkpoint  # noqa: F401  (re-exported helpers)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libflowedge_amd.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_lib = None

EXPORTS = [
    "fe_engine_last_error", "fe_engine_load", "fe_engine_load_with_threads", "fe_weights_load",
    "fe_weights_size_bytes", "fe_weights_free", "fe_engine_create_from_weights",
    "fe_engine_create_from_weights_auto", "fe_engine_thread_count", "fe_engine_cuda_resident",
    "fe_engine_model_metadata", "fe_engine_action_dim", "fe_engine_action_horizon",
    "fe_engine_diffusion_metadata", "fe_engine_condition_dim", "fe_engine_sample_diffusion",
    "fe_engine_diffusion_denoise", "fe_engine_sample_condition", "fe_engine_free",
    "fe_engine_sample_diffusion_batch", "fe_engine_sample_condition_batch",
    "fe_engine_diffusion_denoise_batch", "fe_engine_sample_device", "fe_engine_prepare",
    "fe_engine_max_batch", "fe_engine_device_bytes", "fe_device_alloc_count",
    "fe_engine_last_device_ms", "fe_engine_conv_count", "fe_engine_conv_info",
    "fe_engine_time_convs", "fe_engine_flow_begin", "fe_engine_make_condition_metadata",
    "fe_engine_flow_begin_request", "fe_engine_cancel_before", "fe_engine_flow_advance",
    "fe_engine_flow_action_metadata", "fe_engine_diffusion_begin",
    "fe_engine_diffusion_begin_generation", "fe_engine_diffusion_advance",
    "fe_weights_model_digest", "fe_engine_conv_path", "fe_engine_conv_slices",
    "fe_engine_graph_captures",
    "fe_engine_diffusion_denoise_noalloc", "fe_engine_persistent_tick",
    "fe_engine_persistent_tick_reason", "fe_encoder_load", "fe_encoder_free", "fe_encoder_shape",
    "fe_encoder_encode", "fe_encoder_encode_device", "fe_encoder_last_device_ms",
    "fe_encoder_device_bytes",
]

SCHEDULERS = {"ddim": 0, "ddpm": 1}
SOLVERS = {"euler": 0, "heun": 1, "rk4": 2}


class DiffusionMetadata(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("protocol_version", ctypes.c_uint32),
                ("clip_sample", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("action_dim", ctypes.c_uint64), ("condition_dim", ctypes.c_uint64),
                ("horizon", ctypes.c_uint64), ("action_steps", ctypes.c_uint64),
                ("observation_steps", ctypes.c_uint64), ("train_timesteps", ctypes.c_uint64),
                ("clip_sample_range", ctypes.c_float), ("reserved_float", ctypes.c_float)]


class ModelMetadata(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("protocol_version", ctypes.c_uint32),
                ("architecture", ctypes.c_uint32), ("precision", ctypes.c_uint32),
                ("model_digest", ctypes.c_uint8 * 16), ("d_model", ctypes.c_uint64),
                ("n_layers", ctypes.c_uint64), ("d_inner", ctypes.c_uint64),
                ("d_state", ctypes.c_uint64), ("d_conv", ctypes.c_uint64),
                ("action_dim", ctypes.c_uint64), ("condition_dim", ctypes.c_uint64),
                ("decode_snapshot_bytes", ctypes.c_uint64)]


class ConditionMetadata(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("protocol_version", ctypes.c_uint32),
                ("solver", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("model_digest", ctypes.c_uint8 * 16), ("timestamp_ns", ctypes.c_uint64),
                ("deadline_ns", ctypes.c_uint64), ("generation", ctypes.c_uint64),
                ("condition_dim", ctypes.c_uint64), ("action_dim", ctypes.c_uint64),
                ("solver_steps", ctypes.c_uint64), ("remaining_nfe", ctypes.c_uint64)]


class ActionMetadata(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("protocol_version", ctypes.c_uint32),
                ("solver", ctypes.c_uint32), ("status", ctypes.c_uint32),
                ("model_digest", ctypes.c_uint8 * 16), ("timestamp_ns", ctypes.c_uint64),
                ("deadline_ns", ctypes.c_uint64), ("generation", ctypes.c_uint64),
                ("condition_dim", ctypes.c_uint64), ("action_dim", ctypes.c_uint64),
                ("remaining_nfe", ctypes.c_uint64)]


def lib():
    """The loaded C ABI library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                          "python -m flowedge_amd.build")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, u64, cint = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int
    L.fe_engine_last_error.restype = ctypes.c_char_p
    for name in ("fe_engine_load",):
        getattr(L, name).restype = vp
        getattr(L, name).argtypes = [ctypes.c_char_p]
    L.fe_engine_load_with_threads.restype = vp
    L.fe_engine_load_with_threads.argtypes = [ctypes.c_char_p, ctypes.c_uint]
    L.fe_weights_load.restype = vp
    L.fe_weights_load.argtypes = [ctypes.c_char_p]
    L.fe_weights_size_bytes.restype = sz
    L.fe_weights_size_bytes.argtypes = [vp]
    L.fe_weights_free.argtypes = [vp]
    L.fe_engine_create_from_weights.restype = vp
    L.fe_engine_create_from_weights.argtypes = [vp, ctypes.c_uint]
    L.fe_engine_create_from_weights_auto.restype = vp
    L.fe_engine_create_from_weights_auto.argtypes = [vp]
    L.fe_engine_free.argtypes = [vp]
    L.fe_engine_thread_count.restype = ctypes.c_uint
    L.fe_engine_thread_count.argtypes = [vp]
    L.fe_engine_cuda_resident.argtypes = [vp]
    L.fe_engine_model_metadata.argtypes = [vp, ctypes.POINTER(ModelMetadata)]
    for name in ("fe_engine_action_dim", "fe_engine_action_horizon", "fe_engine_condition_dim",
                 "fe_engine_max_batch", "fe_engine_device_bytes"):
        getattr(L, name).restype = sz
        getattr(L, name).argtypes = [vp]
    L.fe_engine_diffusion_metadata.argtypes = [vp, ctypes.POINTER(DiffusionMetadata)]
    L.fe_engine_sample_diffusion.argtypes = [vp, _f32p, _f32p, sz, cint, u64, _f32p]
    L.fe_engine_diffusion_denoise.argtypes = [vp, _f32p, _f32p, ctypes.c_float, _f32p]
    L.fe_engine_sample_condition.argtypes = [vp, _f32p, _f32p, sz, cint, _f32p]
    L.fe_engine_sample_diffusion_batch.argtypes = [vp, _f32p, _f32p, sz, sz, cint, u64, _f32p]
    L.fe_engine_sample_condition_batch.argtypes = [vp, _f32p, _f32p, sz, sz, cint, _f32p]
    L.fe_engine_diffusion_denoise_batch.argtypes = [vp, _f32p, _f32p, sz, ctypes.c_float, _f32p]
    L.fe_engine_sample_device.argtypes = [vp, cint, vp, vp, sz, sz, cint, u64, vp]
    L.fe_engine_prepare.argtypes = [vp, cint, sz, sz, cint]
    L.fe_engine_diffusion_denoise_noalloc.argtypes = [vp, vp, vp, sz, ctypes.c_float, vp, vp]
    L.fe_device_alloc_count.restype = u64
    L.fe_engine_graph_captures.restype = u64
    L.fe_engine_graph_captures.argtypes = [vp]
    L.fe_engine_persistent_tick.argtypes = [vp]
    L.fe_engine_persistent_tick_reason.restype = ctypes.c_char_p
    L.fe_engine_persistent_tick_reason.argtypes = [vp]
    L.fe_engine_last_device_ms.restype = ctypes.c_float
    L.fe_engine_last_device_ms.argtypes = [vp]
    L.fe_engine_conv_count.argtypes = [vp, ctypes.POINTER(sz)]
    L.fe_engine_conv_info.argtypes = [vp, sz, ctypes.c_char_p, sz, ctypes.POINTER(u64),
                                      ctypes.POINTER(u64)]
    L.fe_engine_time_convs.argtypes = [vp, ctypes.POINTER(sz), sz, sz, sz,
                                       ctypes.POINTER(ctypes.c_float)]
    L.fe_engine_conv_path.argtypes = [vp, sz, sz, ctypes.POINTER(cint)]
    L.fe_engine_conv_slices.argtypes = [vp, sz, sz, ctypes.POINTER(cint)]
    L.fe_engine_flow_begin.argtypes = [vp, _f32p, _f32p, sz, cint]
    L.fe_engine_make_condition_metadata.argtypes = [vp, u64, u64, u64, sz, cint,
                                                    ctypes.POINTER(ConditionMetadata)]
    L.fe_engine_flow_begin_request.argtypes = [vp, _f32p, _f32p,
                                               ctypes.POINTER(ConditionMetadata)]
    L.fe_engine_cancel_before.restype = None
    L.fe_engine_cancel_before.argtypes = [vp, u64]
    L.fe_engine_flow_advance.argtypes = [vp, sz, _f32p, ctypes.POINTER(sz)]
    L.fe_engine_flow_action_metadata.argtypes = [vp, ctypes.POINTER(ActionMetadata)]
    L.fe_engine_diffusion_begin.argtypes = [vp, _f32p, _f32p, sz, cint, u64]
    L.fe_engine_diffusion_begin_generation.argtypes = [vp, _f32p, _f32p, sz, cint, u64, u64]
    L.fe_engine_diffusion_advance.argtypes = [vp, sz, _f32p, ctypes.POINTER(sz)]
    L.fe_weights_model_digest.argtypes = [vp, ctypes.POINTER(ctypes.c_uint8 * 16)]
    L.fe_encoder_load.restype = vp
    L.fe_encoder_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, sz, sz, sz, sz, sz]
    L.fe_encoder_free.restype = None
    L.fe_encoder_free.argtypes = [vp]
    L.fe_encoder_shape.argtypes = [vp, ctypes.POINTER(sz), ctypes.POINTER(sz), ctypes.POINTER(sz)]
    L.fe_encoder_encode.argtypes = [vp, _f32p, sz, _f32p]
    L.fe_encoder_encode_device.argtypes = [vp, vp, sz, vp, sz, sz]
    L.fe_encoder_last_device_ms.restype = ctypes.c_float
    L.fe_encoder_last_device_ms.argtypes = [vp]
    L.fe_encoder_device_bytes.restype = sz
    L.fe_encoder_device_bytes.argtypes = [vp]
    _lib = L
    return L


def last_error() -> str:
    return lib().fe_engine_last_error().decode()


def weights_digest(path: str) -> str:
    """Model digest (hex) of a checkpoint, computed on the host without a GPU."""
    L = lib()
    w = L.fe_weights_load(path.encode())
    if not w:
        raise RuntimeError(last_error())
    try:
        d = (ctypes.c_uint8 * 16)()
        if L.fe_weights_model_digest(w, ctypes.byref(d)) != 0:
            raise RuntimeError(last_error())
        return _digest_hex(d)
    finally:
        L.fe_weights_free(w)


def device_alloc_count() -> int:
    return int(lib().fe_device_alloc_count())


def _arr(a, shape=None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    if shape is not None and a.size != int(np.prod(shape)):
        raise RuntimeError(f"expected {int(np.prod(shape))} values, got {a.size}")
    return a


def _p(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def _digest_hex(d) -> str:
    return bytes(d).hex()


class Engine:
    """One loaded Diffusion Policy checkpoint, device-resident on the current GPU."""

    def __init__(self, path: str, threads: int | None = None):
        L = lib()
        h = (L.fe_engine_load(path.encode()) if threads is None else
             L.fe_engine_load_with_threads(path.encode(), int(threads)))
        if not h:
            raise RuntimeError(last_error())
        self._h = h
        md = DiffusionMetadata()
        if L.fe_engine_diffusion_metadata(self._h, ctypes.byref(md)) != 0:
            raise RuntimeError(last_error())
        self._md = md

    def close(self):
        if getattr(self, "_h", None):
            lib().fe_engine_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may already be unloaded
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- properties (flowedge_ext.cc:793-800) ----
    @property
    def action_dim(self) -> int:
        return int(lib().fe_engine_action_dim(self._h))

    @property
    def action_horizon(self) -> int:
        return int(lib().fe_engine_action_horizon(self._h))

    @property
    def condition_dim(self) -> int:
        return int(lib().fe_engine_condition_dim(self._h))

    @property
    def thread_count(self) -> int:
        return int(lib().fe_engine_thread_count(self._h))

    @property
    def cuda_resident(self) -> bool:
        return bool(lib().fe_engine_cuda_resident(self._h))

    @property
    def diffusion_metadata(self) -> dict:
        md = self._md
        return {f: getattr(md, f) for f, _ in DiffusionMetadata._fields_ if "reserved" not in f}

    @property
    def model_metadata(self) -> dict:
        mm = ModelMetadata()
        if lib().fe_engine_model_metadata(self._h, ctypes.byref(mm)) != 0:
            raise RuntimeError(last_error())
        return {"protocol_version": mm.protocol_version, "architecture": mm.architecture,
                "precision": mm.precision, "model_digest": _digest_hex(mm.model_digest),
                "d_model": mm.d_model, "n_layers": mm.n_layers, "action_dim": mm.action_dim,
                "action_horizon": self.action_horizon, "condition_dim": mm.condition_dim,
                "decode_snapshot_bytes": mm.decode_snapshot_bytes}

    @property
    def max_batch(self) -> int:
        return int(lib().fe_engine_max_batch(self._h))

    @property
    def device_bytes(self) -> int:
        return int(lib().fe_engine_device_bytes(self._h))

    @property
    def persistent_tick(self) -> bool:
        """Batch-1 ticks run as one persistent kernel launch (else per-layer graphs)."""
        return bool(lib().fe_engine_persistent_tick(self._h))

    @property
    def persistent_tick_reason(self) -> str:
        return lib().fe_engine_persistent_tick_reason(self._h).decode()

    @property
    def graph_captures(self) -> int:
        return int(lib().fe_engine_graph_captures(self._h))

    @property
    def last_device_ms(self) -> float:
        return float(lib().fe_engine_last_device_ms(self._h))

    def _values(self) -> int:
        return self.action_horizon * self.action_dim

    def _check(self, rc: int):
        if rc != 0:
            raise RuntimeError(last_error())

    # ---- Diffusion Policy (flowedge_ext.cc:518-561, 837-847) ----
    def sample_diffusion(self, condition, noise, steps: int = 10, scheduler: str = "ddim",
                         seed: int = 0) -> np.ndarray:
        out = np.empty((self.action_horizon, self.action_dim), np.float32)
        self.sample_diffusion_into(condition, noise, out, steps, scheduler, seed)
        return out

    def sample_diffusion_into(self, condition, noise, output, steps: int = 10,
                              scheduler: str = "ddim", seed: int = 0) -> None:
        c = _arr(condition, (self.condition_dim,))
        n = _arr(noise, (self._values(),))
        if not (isinstance(output, np.ndarray) and output.dtype == np.float32 and
                output.flags["C_CONTIGUOUS"] and output.size == self._values()):
            raise RuntimeError("output must be a contiguous float32 array of horizon*action_dim")
        if scheduler not in SCHEDULERS:
            raise RuntimeError("scheduler must be 'ddim' or 'ddpm'")
        self._check(lib().fe_engine_sample_diffusion(self._h, _p(c), _p(n), steps,
                                                     SCHEDULERS[scheduler], seed, _p(output)))

    def diffusion_denoise(self, condition, sample, timestep: float) -> np.ndarray:
        c = _arr(condition, (self.condition_dim,))
        s = _arr(sample, (self._values(),))
        out = np.empty((self.action_horizon, self.action_dim), np.float32)
        self._check(lib().fe_engine_diffusion_denoise(self._h, _p(c), _p(s), float(timestep),
                                                      _p(out)))
        return out

    def sample_condition(self, condition, noise, output, steps: int = 10,
                         method: str = "euler") -> None:
        c = _arr(condition, (self.condition_dim,))
        n = _arr(noise, (self._values(),))
        self._output(output)
        if method not in SOLVERS:
            raise RuntimeError("method must be 'euler', 'heun' or 'rk4'")
        self._check(lib().fe_engine_sample_condition(self._h, _p(c), _p(n), steps,
                                                     SOLVERS[method], _p(output)))

    # ---- resumable solves (flowedge_ext.cc:564-623, 848-856) ----
    def _output(self, output) -> None:
        if not (isinstance(output, np.ndarray) and output.dtype == np.float32 and
                output.flags["C_CONTIGUOUS"] and output.size == self._values()):
            raise RuntimeError("output must be a contiguous float32 array of horizon*action_dim")

    def flow_begin(self, condition, noise, steps: int = 10, method: str = "euler",
                   generation: int | None = None, timestamp_ns: int = 0,
                   deadline_ns: int = 0) -> None:
        """Begin a resumable flow solve; with `generation`, a cancellable versioned request."""
        c = _arr(condition, (self.condition_dim,))
        n = _arr(noise, (self._values(),))
        if method not in SOLVERS:
            raise RuntimeError("method must be one of: euler, heun, rk4")
        L = lib()
        if generation is None:
            self._check(L.fe_engine_flow_begin(self._h, _p(c), _p(n), steps, SOLVERS[method]))
            return
        md = ConditionMetadata()
        self._check(L.fe_engine_make_condition_metadata(self._h, timestamp_ns, deadline_ns,
                                                        generation, steps, SOLVERS[method],
                                                        ctypes.byref(md)))
        self._check(L.fe_engine_flow_begin_request(self._h, _p(c), _p(n), ctypes.byref(md)))

    def flow_advance(self, output, step_budget: int = 1) -> int:
        """Run at most `step_budget` solver steps into `output`; returns the steps remaining."""
        self._output(output)
        rem = ctypes.c_size_t()
        self._check(lib().fe_engine_flow_advance(self._h, step_budget, _p(output),
                                                 ctypes.byref(rem)))
        return int(rem.value)

    def cancel_before(self, generation: int) -> None:
        lib().fe_engine_cancel_before(self._h, generation)

    @property
    def flow_metadata(self) -> dict:
        md = ActionMetadata()
        self._check(lib().fe_engine_flow_action_metadata(self._h, ctypes.byref(md)))
        return {"protocol_version": md.protocol_version, "solver": md.solver,
                "status": md.status, "model_digest": _digest_hex(md.model_digest),
                "timestamp_ns": md.timestamp_ns, "deadline_ns": md.deadline_ns,
                "generation": md.generation, "condition_dim": md.condition_dim,
                "action_dim": md.action_dim, "remaining_nfe": md.remaining_nfe}

    def diffusion_begin(self, condition, noise, steps: int = 10, scheduler: str = "ddim",
                        seed: int = 0, generation: int | None = None) -> None:
        """Begin a resumable DDIM/DDPM solve (extension); cancellable with `generation`."""
        c = _arr(condition, (self.condition_dim,))
        n = _arr(noise, (self._values(),))
        if scheduler not in SCHEDULERS:
            raise RuntimeError("scheduler must be 'ddim' or 'ddpm'")
        L = lib()
        if generation is None:
            self._check(L.fe_engine_diffusion_begin(self._h, _p(c), _p(n), steps,
                                                    SCHEDULERS[scheduler], seed))
        else:
            self._check(L.fe_engine_diffusion_begin_generation(
                self._h, _p(c), _p(n), steps, SCHEDULERS[scheduler], seed, generation))

    def diffusion_advance(self, output, step_budget: int = 1) -> int:
        self._output(output)
        rem = ctypes.c_size_t()
        self._check(lib().fe_engine_diffusion_advance(self._h, step_budget, _p(output),
                                                      ctypes.byref(rem)))
        return int(rem.value)

    # ---- batched extensions ----
    def _batch(self, condition) -> tuple[np.ndarray, int]:
        c = _arr(condition)
        b = c.size // self.condition_dim
        if b < 1 or c.size != b * self.condition_dim:
            raise RuntimeError(f"condition must hold whole rows of {self.condition_dim} values")
        return c, b

    def sample_diffusion_batch(self, condition, noise, steps: int = 10, scheduler: str = "ddim",
                               seed: int = 0) -> np.ndarray:
        c, b = self._batch(condition)
        n = _arr(noise, (b * self._values(),))
        out = np.empty((b, self.action_horizon, self.action_dim), np.float32)
        self._check(lib().fe_engine_sample_diffusion_batch(self._h, _p(c), _p(n), b, steps,
                                                           SCHEDULERS[scheduler], seed, _p(out)))
        return out

    def sample_condition_batch(self, condition, noise, steps: int = 10,
                               method: str = "euler") -> np.ndarray:
        c, b = self._batch(condition)
        n = _arr(noise, (b * self._values(),))
        out = np.empty((b, self.action_horizon, self.action_dim), np.float32)
        self._check(lib().fe_engine_sample_condition_batch(self._h, _p(c), _p(n), b, steps,
                                                           SOLVERS[method], _p(out)))
        return out

    def diffusion_denoise_batch(self, condition, sample, timestep: float) -> np.ndarray:
        c, b = self._batch(condition)
        s = _arr(sample, (b * self._values(),))
        out = np.empty((b, self.action_horizon, self.action_dim), np.float32)
        self._check(lib().fe_engine_diffusion_denoise_batch(self._h, _p(c), _p(s), b,
                                                            float(timestep), _p(out)))
        return out

    def sample_device(self, kind: int, cond_ptr: int, noise_ptr: int, batch: int, steps: int,
                      mode: int, seed: int, action_ptr: int) -> None:
        """Device-resident sampling: the pointers are device addresses (e.g. tensor.data_ptr())."""
        self._check(lib().fe_engine_sample_device(self._h, kind, cond_ptr, noise_ptr, batch,
                                                  steps, mode, seed, action_ptr))

    def denoise_noalloc(self, cond_ptr: int, sample_ptr: int, batch: int, timestep: float,
                        out_ptr: int, stream: int | None = None) -> None:
        """Allocation-free batched denoise on device pointers (static device scratch); with
        `stream` (a hipStream_t handle) it is only enqueued."""
        self._check(lib().fe_engine_diffusion_denoise_noalloc(
            self._h, cond_ptr, sample_ptr, batch, float(timestep), out_ptr, stream))

    def prepare(self, kind: int, batch: int, steps: int, mode: int) -> None:
        self._check(lib().fe_engine_prepare(self._h, kind, batch, steps, mode))

    def convolutions(self) -> list[dict]:
        """The fused convolutions of one U-Net evaluation in launch order: name and algorithmic
        bytes (weights + biases per launch, activations + per-channel parameters per sample)."""
        L = lib()
        n = ctypes.c_size_t()
        self._check(L.fe_engine_conv_count(self._h, ctypes.byref(n)))
        out = []
        buf = ctypes.create_string_buffer(256)
        wb, sb = ctypes.c_uint64(), ctypes.c_uint64()
        for i in range(n.value):
            self._check(L.fe_engine_conv_info(self._h, i, buf, 256, ctypes.byref(wb),
                                              ctypes.byref(sb)))
            out.append({"index": i, "name": buf.value.decode(), "weight_bytes": wb.value,
                        "sample_bytes": sb.value})
        return out

    def conv_paths(self, batch: int = 1) -> list[str]:
        """Kernels each convolution of convolutions() runs on at `batch`: "fused"
        (weight-streaming), "matrix" (matrix-core implicit GEMM) or "general" (general-shape)."""
        L = lib()
        n = ctypes.c_size_t()
        self._check(L.fe_engine_conv_count(self._h, ctypes.byref(n)))
        names = ("fused", "matrix", "general")
        out = []
        p = ctypes.c_int()
        for i in range(n.value):
            self._check(L.fe_engine_conv_path(self._h, i, batch, ctypes.byref(p)))
            out.append(names[p.value])
        return out

    def conv_slices(self, batch: int = 1) -> list[int]:
        """Input-channel slices each convolution of convolutions() runs with at `batch` (1:
        unsliced)."""
        L = lib()
        n = ctypes.c_size_t()
        self._check(L.fe_engine_conv_count(self._h, ctypes.byref(n)))
        out = []
        p = ctypes.c_int()
        for i in range(n.value):
            self._check(L.fe_engine_conv_slices(self._h, i, batch, ctypes.byref(p)))
            out.append(p.value)
        return out

    def time_convolutions(self, indices, batch: int = 1, iters: int = 100) -> float:
        """Mean device time (microseconds) of one launch of the given convolutions, launched
        round-robin on the engine's stream."""
        idx = (ctypes.c_size_t * len(indices))(*indices)
        us = ctypes.c_float()
        self._check(lib().fe_engine_time_convs(self._h, idx, len(indices), batch, iters,
                                               ctypes.byref(us)))
        return float(us.value)
