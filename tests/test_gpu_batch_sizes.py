"""Oracle parity at the batch sizes the benchmark reports, on every sample.

A batch is defined as B independent batch-1 calls (the reference's engine has no batch argument:
src/core/api/engine.h:93-97; diffusion.cc:916-1035 samples one condition), so the oracle result is
`oracle.sample_batch`, B independent CPU samples spread over worker threads.  These batches run
the matrix-core implicit GEMMs with the tile shapes and split-K choices of their own size, which
is why they are checked at exactly these sizes: pusht-size DDIM-10 at B=256 (F32), the bimanual
BF16 U-Net at B=64 and the flow U-Net at B=128 with RK4-4 and Euler-10.  Tolerance: max |err|
<= 1e-4 in action units (action scale 1) for fp32 weights; the BF16-weight model is held to the
same 1e-4 because the oracle runs on the identical BF16-rounded weights (contract bound 2e-2).
"""

from __future__ import annotations

import time

import numpy as np
import pytest

import flowedge_amd
import oracle
from flowedge_amd import checkpoint as ck

pytestmark = pytest.mark.gpu

TOL = 1e-4
WORKERS = 16


def say(msg: str):
    print(msg, flush=True)


def maxerr(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def check_all(got, want, label):
    err = np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)), axis=(1, 2))
    worst = int(np.argmax(err))
    say(f"{label}: max |err| {err[worst]:.3e} (sample {worst} of {len(err)})")
    assert np.all(np.isfinite(got))
    assert err[worst] <= TOL


def test_pusht_b256_ddim10(ckpt_dir, monkeypatch):
    spec = ck.SPECS["pusht"]
    path = ck.cached_checkpoint("pusht", ckpt_dir)
    B = 256
    cond, noise = ck.inputs(spec, batch=B)
    say(f"pusht DDIM-10 B={B}: GPU")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_diffusion_batch(cond, noise, steps=10)
    # The opt-in split-F32 path (F32 operands as BF16 hi + lo terms on the BF16 matrix cores)
    # at the same batch, against the same oracle samples.
    monkeypatch.setenv("FLOWEDGE_MFMA_F32_SPLIT", "1")
    with flowedge_amd.Engine(path) as e:
        got_split = e.sample_diffusion_batch(cond, noise, steps=10)
    t0 = time.time()
    want = oracle.Oracle(path).sample_batch(cond, noise, 10, workers=WORKERS)
    say(f"pusht DDIM-10 B={B}: oracle {time.time() - t0:.1f} s")
    check_all(got, want, f"pusht DDIM-10 B={B}")
    assert np.all(got >= -1.0) and np.all(got <= 1.0)
    check_all(got_split, want, f"pusht DDIM-10 B={B} split-F32")


def test_bimanual_bf16_b64_ddim10(ckpt_dir):
    spec = ck.SPECS["bimanual"]
    path = ck.cached_checkpoint("bimanual", ckpt_dir)
    B = 64
    cond, noise = ck.inputs(spec, batch=B)
    say(f"bimanual BF16 DDIM-10 B={B}: GPU")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_diffusion_batch(cond, noise, steps=10)
    want = oracle.Oracle(path).sample_batch(cond, noise, 10, workers=WORKERS)
    check_all(got, want, f"bimanual DDIM-10 B={B}")


@pytest.mark.parametrize("method,steps", [("rk4", 4), ("euler", 10)])
def test_flow_b128(ckpt_dir, method, steps):
    spec = ck.SPECS["flow"]
    path = ck.cached_checkpoint("flow", ckpt_dir)
    B = 128
    cond, x0 = ck.inputs(spec, batch=B)
    say(f"flow {method}-{steps} B={B}: GPU")
    with flowedge_amd.Engine(path) as e:
        got = e.sample_condition_batch(cond, x0, steps=steps, method=method)
    t0 = time.time()
    want = oracle.Oracle(path).sample_batch(cond, x0, steps, 1, flowedge_amd.SOLVERS[method],
                                            workers=WORKERS)
    say(f"flow {method}-{steps} B={B}: oracle {time.time() - t0:.1f} s")
    check_all(got, want, f"flow {method}-{steps} B={B}")
