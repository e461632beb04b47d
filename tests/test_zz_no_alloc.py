"""The allocation-free denoise entry point against fe_engine_diffusion_denoise_batch.

fe_engine_diffusion_denoise_noalloc runs one U-Net evaluation with its whole workspace in the
library's static device scratch array (no device allocation, no graph capture), on device
pointers.  Its output must match the existing batched denoise entry point on the same inputs to
the fp32 bound (max |err| <= 1e-4 in action units; batches below the matrix-core threshold run the
same kernels and agree bit for bit), on two calls in a row, the second with a smaller batch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import flowedge_amd
from flowedge_amd import checkpoint as ck

pytestmark = pytest.mark.gpu

TOL = 1e-4


def say(msg: str):
    print(msg, flush=True)


def noalloc_fn():
    lib = flowedge_amd.lib()
    fn = lib.fe_engine_diffusion_denoise_noalloc
    vp = ctypes.c_void_p
    fn.argtypes = [vp, vp, vp, ctypes.c_size_t, ctypes.c_float, vp, vp]
    fn.restype = ctypes.c_int
    return fn


def maxerr(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


@pytest.mark.parametrize("workload,batches", [("tiny", (9, 3)), ("pusht", (3, 1))])
def test_noalloc_denoise_matches_denoise_batch(ckpt_dir, workload, batches):
    import torch

    fn = noalloc_fn()
    spec = ck.SPECS[workload]
    path = ck.cached_checkpoint(workload, ckpt_dir)
    dev = torch.device("cuda:0")
    with flowedge_amd.Engine(path) as e:
        for call, (batch, t) in enumerate(zip(batches, (61.0, 7.0))):
            cond, x = ck.inputs(spec, batch=batch, cond_seed=11 + call, noise_seed=12 + call)
            want = e.diffusion_denoise_batch(cond, x, t)
            dc = torch.from_numpy(cond).to(dev)
            dx = torch.from_numpy(x).to(dev)
            out = torch.full((batch, spec.horizon, spec.action_dim), float("nan"),
                             dtype=torch.float32, device=dev)
            torch.cuda.synchronize()
            allocs = flowedge_amd.device_alloc_count()
            captures = e.graph_captures
            free0 = torch.cuda.mem_get_info()[0]
            say(f"{workload} noalloc denoise B={batch} t={t}")
            rc = fn(e._h, dc.data_ptr(), dx.data_ptr(), batch, t, out.data_ptr(), None)
            assert rc == 0, flowedge_amd.last_error()
            got = out.cpu().numpy()
            err = maxerr(got, want)
            say(f"{workload} noalloc B={batch}: max |err| vs denoise_batch {err:.3e}")
            assert np.all(np.isfinite(got)) and err <= TOL
            if batch < 4:  # the same fused kernels as the arena path
                assert np.array_equal(got, want)
            assert flowedge_amd.device_alloc_count() == allocs
            assert e.graph_captures == captures
            assert torch.cuda.mem_get_info()[0] == free0
            # On a caller's stream: enqueued only, complete after the stream synchronises.
            out2 = torch.full_like(out, float("nan"))
            torch.cuda.synchronize()
            s = torch.cuda.Stream()
            rc = fn(e._h, dc.data_ptr(), dx.data_ptr(), batch, t, out2.data_ptr(),
                    ctypes.c_void_p(s.cuda_stream))
            assert rc == 0, flowedge_amd.last_error()
            s.synchronize()
            assert np.array_equal(out2.cpu().numpy(), got)


def test_noalloc_rejects_oversized_batch_and_bad_arguments(ckpt_dir):
    import torch

    fn = noalloc_fn()
    spec = ck.SPECS["pusht"]
    path = ck.cached_checkpoint("pusht", ckpt_dir)
    dev = torch.device("cuda:0")
    buf = torch.zeros(1024, dtype=torch.float32, device=dev)
    p = buf.data_ptr()
    with flowedge_amd.Engine(path) as e:
        # 256 pusht-size samples need far more than the scratch array holds: refused before any
        # work is enqueued (the device buffers passed here would be too small for it).
        assert fn(e._h, p, p, 256, 5.0, p, None) == 1
        assert "scratch" in flowedge_amd.last_error()
        assert fn(e._h, p, p, 0, 5.0, p, None) == 1
        assert fn(e._h, p, p, 1, float("nan"), p, None) == 1
        assert fn(e._h, None, p, 1, 5.0, p, None) == 1
        assert spec.horizon * spec.action_dim <= buf.numel()
