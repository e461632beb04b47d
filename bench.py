#!/usr/bin/env python3
"""Benchmark of the Diffusion Policy U-Net sampling tick on one MI355X.

Headline (``value``): p50 latency of one sampling tick -- 10-step DDIM of the LeRobot
diffusion_pusht-size Conv1D U-Net (widths 512/1024/2048, horizon 16, action_dim 2, condition
132, fp32) at batch 1 -- with condition and noise already resident in HBM.  A "step" of this
benchmark is one tick.  Also reported: host-to-host p50/p99 through the host-pointer ABI
(PCIe-inclusive, never ``value``), actions/sec at batch 256, the HBM roofline of the tick, and the
CPU oracle timed on this host's cores.

Roofline (``roofline``): the dominant kernel of the tick, i.e. the fused convolution shape with
the largest device time per U-Net evaluation (the 2048<-2048, K=5, L=4 convolution with the
GroupNorm+Mish+FiLM prologue, 4 launches per evaluation).  Its algorithmic bytes per launch are
its weights and biases once plus its input/output activations and per-channel parameters once
(83.9 MB); ``achieved`` = those bytes / the mean launch duration, timed with hipEvents on the
engine's stream over launches that cycle through its distinct layers (336 MB of weights, more
than the 256 MB MALL, as in a tick).  ``tick_roofline`` gives the same ratio for a whole tick:
all U-Net weights once per evaluation (1,006,047,844 B x 10) / the device time of one graph
replay.  ``traffic`` is the HBM bytes per launch measured with rocprofv3 PMC counters (read from
the committed summary when present).  ``python bench.py --roofline-only`` runs just that kernel
loop (plus a 256 MiB copy used to calibrate the counters) for profiling.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0  # dense
METRIC = "p50 tick latency (B=1, 10-step DDIM) + actions/sec at B=256, % roofline"


def unet_bytes_and_flops(spec, batch: int = 1):
    """Algorithmic bytes (each weight once) and FLOPs of one U-Net evaluation."""
    from flowedge_amd import checkpoint as ck

    weight_bytes = 0
    flops = 0
    H = spec.horizon
    dims = list(spec.dims)
    for name, shape, kind, _ in ck.layout(spec):
        n = 1
        for s in shape:
            n *= s
        esize = 2 if (spec.bf16_weights and kind == "w") else 4
        weight_bytes += n * esize
    weight_bytes += (2 * spec.action_dim + 16 + len(dims)) * 4  # action range, meta, dims

    def conv_f(oc, ic, k, lout):
        return 2 * oc * ic * k * lout

    L = H
    for s, oc in enumerate(dims):
        ic = spec.action_dim if s == 0 else dims[s - 1]
        for blk in range(2):
            cin = ic if blk == 0 else oc
            flops += conv_f(oc, cin, spec.kernel, L) + conv_f(oc, oc, spec.kernel, L)
            flops += 2 * (2 * oc) * (spec.timestep_dim + spec.cond_dim)
            if cin != oc:
                flops += conv_f(oc, cin, 1, L)
        if s + 1 < len(dims):
            flops += conv_f(oc, oc, 3, L // 2)
            L //= 2
    for _ in range(2):
        flops += 2 * conv_f(dims[-1], dims[-1], spec.kernel, L) + 2 * 2 * dims[-1] * (
            spec.timestep_dim + spec.cond_dim)
    for u in range(len(dims) - 1):
        high, low = dims[-1 - u], dims[-2 - u]
        flops += conv_f(low, 2 * high, spec.kernel, L) + conv_f(low, 2 * high, 1, L)
        flops += 3 * conv_f(low, low, spec.kernel, L) + 2 * 2 * (2 * low) * (
            spec.timestep_dim + spec.cond_dim)
        flops += 2 * low * low * 4 * L  # ConvTranspose K4 over L inputs
        L *= 2
    flops += conv_f(dims[0], dims[0], spec.kernel, H) + conv_f(spec.action_dim, dims[0], 1, H)
    return weight_bytes, flops * batch


DOMINANT_SHAPE = "[2048<-2048 K5 L4 film]"
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "conv_film_2048x2048_L4_pusht_traffic.txt")


def shape_of(name: str) -> str:
    return name[name.index("["):] if "[" in name else name


def conv_flops(shape: str) -> int:
    """FLOPs of one sample through a convolution named "[oc<-ic Kk Llin (down|up)? ... (+1x1)?]"."""
    f = shape.strip("[]").split()
    oc, ic = (int(v) for v in f[0].split("<-"))
    k, lin = int(f[1][1:]), int(f[2][1:])
    lout = lin // 2 if "down" in f else (2 * lin if "up" in f else lin)
    flops = 2 * oc * ic * k * (lin if "up" in f else lout)  # ConvT: 2*OC*IC*K*L_in
    if "+1x1" in f:
        flops += 2 * oc * ic * lout
    return flops


def conv_breakdown(eng, batch: int = 1, iters: int = 50):
    """Mean launch time of every convolution shape of one U-Net evaluation (each shape's distinct
    layers launched round-robin, on the kernels a call of this batch uses) and its share of an
    evaluation."""
    convs = eng.convolutions()
    slices = eng.conv_slices(batch)
    groups = {}
    for c in convs:
        groups.setdefault(shape_of(c["name"]), []).append(c)
    rows = []
    for shape, cs in groups.items():
        us = eng.time_convolutions([c["index"] for c in cs], batch=batch, iters=iters)
        nbytes = cs[0]["weight_bytes"] + cs[0]["sample_bytes"] * batch
        row = {"shape": shape, "launches_per_nfe": len(cs), "us_per_launch": round(us, 3),
               "slices": sorted({slices[c["index"]] for c in cs}),
               "us_per_nfe": round(us * len(cs), 2), "bytes_per_launch": nbytes,
               "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "indices": [c["index"] for c in cs]}
        if batch > 1:
            row["tflops"] = round(conv_flops(shape) * batch / (us * 1e-6) / 1e12, 2)
        rows.append(row)
    rows.sort(key=lambda r: -r["us_per_nfe"])
    return rows


def encoder_timing(n: int, iters: int = 30) -> dict:
    """The observation encoder (resnet18-GroupNorm + keypoints, fe_encoder_encode) on n synthetic
    96 x 96 camera images center-cropped to 84 x 84: device time of its graph (hipEvents)."""
    import numpy as np

    from flowedge_amd import checkpoint as ck
    from flowedge_amd.encoder import RgbEncoder

    spec = ck.EncoderSpec()
    images = ck.encoder_images(spec, n)
    with RgbEncoder(ck.cached_encoder(), max_images=max(n, 8)) as e:
        for _ in range(3):
            e.encode(images)
        ts = []
        for _ in range(iters):
            e.encode(images)
            ts.append(e.last_device_ms)
    p50 = float(np.median(ts))
    return {"images": n, "image_hw": list(spec.image_hw), "crop_hw": list(spec.crop_hw),
            "keypoints": spec.keypoints, "device_p50_ms": round(p50, 4),
            "us_per_image": round(p50 * 1e3 / n, 2),
            "definition": "fe_encoder_encode on host images; device time of the encoder's graph "
                          "(hipEvents), synthetic LeRobot-named weights"}


def dominant_roofline(eng, iters: int):
    """Live measurement of the dominant convolution (hipEvents around `iters` rounds)."""
    convs = [c for c in eng.convolutions() if shape_of(c["name"]) == DOMINANT_SHAPE]
    if not convs:
        return None
    idx = [c["index"] for c in convs]
    slices = sorted({eng.conv_slices(1)[i] for i in idx})
    kernel = (f"conv_slice_kernel<kConvSame, K=5, LIN=4, kProFilm, RES=false> {DOMINANT_SHAPE}, "
              f"{slices} input-channel slices" if slices != [1] else
              f"conv_kernel<kConvSame, K=5, LIN=4, VEC=4, kProFilm, RES=false> {DOMINANT_SHAPE}")
    us = eng.time_convolutions(idx, batch=1, iters=iters)
    nbytes = convs[0]["weight_bytes"] + convs[0]["sample_bytes"]
    achieved = nbytes / (us * 1e-6) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_PROFILE):
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(line.split(":", 1)[1].strip())
    return {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "traffic_source": ("rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this loop, calibrated on a "
                           "256 MiB copy; read from " + os.path.relpath(TRAFFIC_PROFILE, ROOT))
        if traffic is not None else None,
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "kernel": kernel,
        "algorithmic_bytes_per_launch": nbytes,
        "us_per_launch": round(us, 3),
        "launches_timed": iters * len(idx),
        "layers_cycled": [c["name"] for c in convs],
    }


EXTRA_CONFIGS = [
    # (workload, batch, kind 0 = DDIM / 1 = flow ODE, steps, mode, U-Net evaluations per step, label)
    ("bimanual", 1, 0, 10, 0, 1, "4a: bimanual-size BF16 (H8, A14, cond 1052), B=1, DDIM-10"),
    ("bimanual", 64, 0, 10, 0, 1, "4b: bimanual-size BF16, B=64, DDIM-10"),
    ("flow", 1, 1, 4, 2, 4, "5: flow U-Net (A7, cond 256), B=1, RK4-4"),
    ("flow", 1, 1, 10, 0, 1, "5: flow U-Net, B=1, Euler-10"),
    ("flow", 128, 1, 4, 2, 4, "5b: flow U-Net, B=128, RK4-4"),
    ("flow", 128, 1, 10, 0, 1, "5b: flow U-Net, B=128, Euler-10"),
]


def extra_configs(iters: int = 10, check: bool = True):
    """Device time of the other configurations of the path (one graph replay each)."""
    import numpy as np
    import torch

    import flowedge_amd
    from flowedge_amd import checkpoint as ck

    dev = torch.device("cuda:0")
    engines = {}
    rows = []
    for work, batch, kind, steps, mode, per_step, label in EXTRA_CONFIGS:
        spec = ck.SPECS[work]
        if work not in engines:
            engines[work] = flowedge_amd.Engine(ck.cached_checkpoint(work))
        e = engines[work]
        cond, noise = ck.inputs(spec, batch=batch)
        dc, dn = torch.from_numpy(cond).to(dev), torch.from_numpy(noise).to(dev)
        do = torch.empty((batch, spec.horizon, spec.action_dim), dtype=torch.float32, device=dev)
        e.prepare(kind, batch, steps, mode)
        for _ in range(3):
            e.sample_device(kind, dc.data_ptr(), dn.data_ptr(), batch, steps, mode, 0, do.data_ptr())
        ts = []
        for _ in range(iters):
            e.sample_device(kind, dc.data_ptr(), dn.data_ptr(), batch, steps, mode, 0, do.data_ptr())
            ts.append(e.last_device_ms)
        ms = float(np.median(ts))
        wbytes, nfe_flops = unet_bytes_and_flops(spec)
        nfe = steps * per_step
        gbs = wbytes * nfe / (ms * 1e-3) / 1e9
        tflops = nfe_flops * batch * nfe / (ms * 1e-3) / 1e12
        row = {"config": label, "device_p50_ms": round(ms, 3), "nfe": nfe,
               "actions_per_sec": round(batch * spec.horizon / (ms * 1e-3), 1),
               "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
               "tflops": round(tflops, 2), "finite": bool(torch.isfinite(do).all().item())}
        if check:
            idx = sorted({0, batch // 2, batch - 1})
            row["max_abs_err_vs_oracle"] = oracle_check(ck.cached_checkpoint(work), cond, noise,
                                                        do.cpu().numpy(), steps, idx, kind, mode)
            row["oracle_samples"] = idx
        # The engine's default matrix-core thresholds: 4 samples (F32 weights), 5 (BF16).
        if batch >= 5 and spec.bf16_weights:
            # BF16 weights on the BF16 matrix cores, input split in two terms: two MFMA
            # products per useful product.
            row["mfma"] = "bf16 (2 products per multiply)"
            row["mfma_frac"] = round(2 * tflops / BF16_MFMA_PEAK_TFLOPS, 4)
        elif batch >= 4 and not spec.bf16_weights:
            row["mfma"] = "fp32"
            row["mfma_frac"] = round(tflops / FP32_MFMA_PEAK_TFLOPS, 4)
        rows.append(row)
        print(f"[bench] {label}: {ms:.3f} ms  ({gbs:.0f} GB/s weights, {tflops:.1f} TFLOP/s)",
              file=sys.stderr, flush=True)
    for e in engines.values():
        e.close()
    return rows


def percentile(xs, q):
    import numpy as np

    return float(np.percentile(np.asarray(xs, dtype=np.float64), q))


def cpu_info() -> dict:
    """CPU model and the core counts this process can use."""
    info = {"hardware_concurrency": os.cpu_count() or 1}
    try:
        for line in subprocess.run(["lscpu"], capture_output=True, text=True).stdout.splitlines():
            if line.startswith("Model name"):
                info["model"] = line.split(":", 1)[1].strip()
            elif line.startswith("Socket(s)"):
                info["sockets"] = line.split(":", 1)[1].strip()
    except Exception:
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                info["proc_model_name"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    info.setdefault("model", info.get("proc_model_name", platform.processor() or "unknown"))
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except AttributeError:
        info["affinity"] = info["hardware_concurrency"]
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if quota != "max":
            info["cgroup_cpus"] = round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        pass
    return info


# Worker threads on the GPU host: its CPU share for one GPU is 16 cores, whatever the machine's
# hardware_concurrency is (larger pools only oversubscribe that share).
CPU_SHARE = 16


def cpu_baseline(path, spec, budget_s: float):
    """The CPU oracle (this repository's C++ restatement of the reference CPU path) on the host,
    timed with a steady clock around whole samples as bench/kernels/diffusion_breakdown.cc:35-49
    does: caller thread only, the reference's 8-worker cap (engine_runtime.h:39), all the cores
    this process may use, and the batch-256 configuration extrapolated from a subset of samples
    run as independent engines over shared weights (the reference's batching model,
    engine.h:93-97)."""
    import numpy as np

    import oracle
    from flowedge_amd import checkpoint as ck

    info = cpu_info()
    share = max(1, min(info["affinity"], int(info.get("cgroup_cpus", CPU_SHARE)), CPU_SHARE))
    cond, noise = ck.inputs(spec)
    out = {"cpu": info, "share": share}
    legs = (("threads1", 0, 0.4), ("threads8", 8, 0.15), ("all_cores", share, 0.15))
    for label, threads, frac in legs:
        o = oracle.Oracle(path, threads=threads)
        o.sample(cond[0], noise[0], 10)  # warmup (first-touch of the weights)
        times = []
        t_start = time.perf_counter()
        while len(times) < 20 and (len(times) < 3 or
                                   time.perf_counter() - t_start < budget_s * frac):
            t0 = time.perf_counter()
            o.sample(cond[0], noise[0], 10)
            times.append((time.perf_counter() - t0) * 1e3)
        o.close()
        out[label] = {"p50_ms": percentile(times, 50), "p99_ms": percentile(times, 99),
                      "ticks": len(times), "cores": max(threads, 1)}
    # Batch 256: `share` independent samples at once on `share` workers, scaled to 256 samples.
    cb, nb = ck.inputs(spec, batch=share)
    o = oracle.Oracle(path)
    t0 = time.perf_counter()
    o.sample_batch(cb, nb, 10, workers=share)
    per_round = (time.perf_counter() - t0) * 1e3
    o.close()
    out["b256_all_cores"] = {"ms": per_round * 256 / share, "cores": share,
                             "sample": f"{share} samples on {share} workers, x {256 / share:g}"}
    out["b256_threads1"] = {"ms": out["threads1"]["p50_ms"] * 256, "cores": 1,
                            "sample": "per-sample p50 at threads=1, x 256"}
    return out


def oracle_check(path, cond, noise, got, steps: int, idx, kind: int = 0, mode: int = 0) -> float:
    """Max |GPU - oracle| over the samples `idx` (B independent oracle samples)."""
    import numpy as np

    import oracle

    o = oracle.Oracle(path)
    want = o.sample_batch(cond[idx], noise[idx], steps, kind, mode, workers=CPU_SHARE)
    o.close()
    return float(np.max(np.abs(got[idx].astype(np.float64) - want.astype(np.float64))))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed ticks")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="pusht")
    ap.add_argument("--large-batch", type=int, default=256)
    ap.add_argument("--large-steps", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=30.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the bimanual and flow configs")
    ap.add_argument("--no-split", action="store_true",
                    help="skip the large batch on the BF16 matrix cores with split F32 operands")
    ap.add_argument("--roofline-iters", type=int, default=200,
                    help="rounds over the dominant convolution's layers")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the dominant-kernel loop and a 256 MiB calibration copy")
    ap.add_argument("--encoder", type=int, metavar="IMAGES",
                    help="only the observation encoder on that many camera images, as JSON")
    ap.add_argument("--breakdown", metavar="WORKLOAD:BATCH",
                    help="only the per-shape convolution timing of one U-Net evaluation at that "
                         "batch (diagnostics and profiling), as JSON")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py runs on one GPU: --gpus {args.gpus} is not supported by this build "
              "(the Diffusion Policy tick is measured on a single MI355X).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import flowedge_amd
    from flowedge_amd import checkpoint as ck

    if args.encoder:
        print(json.dumps({"observation_encoder": encoder_timing(args.encoder, iters=100)}),
              flush=True)
        return

    if args.breakdown:
        work, batch = args.breakdown.split(":")
        eng = flowedge_amd.Engine(ck.cached_checkpoint(work))
        rows = conv_breakdown(eng, batch=int(batch), iters=10)
        for r in rows:
            print(f"[bench] {work} B={batch} {r['shape']:36s} x{r['launches_per_nfe']} "
                  f"{r['us_per_launch']:9.2f} us {r.get('tflops', 0):7.1f} TFLOP/s "
                  f"slices {r['slices']}", file=sys.stderr, flush=True)
        print(json.dumps({"breakdown": work, "batch": int(batch),
                          "rows": [{k: v for k, v in r.items() if k != "indices"} for r in rows]}),
              flush=True)
        eng.close()
        return

    spec = ck.SPECS[args.workload]
    path = ck.cached_checkpoint(args.workload)
    print(f"[bench] checkpoint {path}", file=sys.stderr, flush=True)
    wbytes, nfe_flops = unet_bytes_and_flops(spec)
    steps_ddim = 10
    tick_bytes = wbytes * steps_ddim

    eng = flowedge_amd.Engine(path)
    dev = torch.device("cuda:0")
    if args.roofline_only:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)  # calibration: 256 MiB read + 256 MiB written per launch
        torch.cuda.synchronize()
        roof = dominant_roofline(eng, args.roofline_iters)
        print(json.dumps({"roofline": roof}), flush=True)
        return
    cond, noise = ck.inputs(spec, batch=1)
    d_cond = torch.from_numpy(cond).to(dev)
    d_noise = torch.from_numpy(noise).to(dev)
    d_out = torch.empty((1, spec.horizon, spec.action_dim), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    eng.prepare(0, 1, steps_ddim, 0)

    def tick(b, c, n, o):
        eng.sample_device(0, c.data_ptr(), n.data_ptr(), b, steps_ddim, 0, 0, o.data_ptr())

    for _ in range(args.warmup):
        tick(1, d_cond, d_noise, d_out)
    torch.cuda.synchronize()
    lat, devms = [], []
    t_all = time.perf_counter()
    for _ in range(args.steps):
        t0 = time.perf_counter()
        tick(1, d_cond, d_noise, d_out)
        lat.append((time.perf_counter() - t0) * 1e3)
        devms.append(eng.last_device_ms)
    torch.cuda.synchronize()
    total_ms = (time.perf_counter() - t_all) * 1e3
    p50 = percentile(lat, 50)
    dev_p50 = percentile(devms, 50)
    print(f"[bench] B=1 DDIM-10 tick p50 {p50:.3f} ms (device {dev_p50:.3f} ms)", file=sys.stderr,
          flush=True)

    # Host-to-host (PCIe-inclusive) through the reference-shaped ABI.
    # Five untimed calls first (host buffers and caches warm), then at least 5 timed ones.
    host = []
    for i in range(5 + max(5, min(args.steps, 100))):
        t0 = time.perf_counter()
        eng.sample_diffusion(cond[0], noise[0], steps=steps_ddim)
        host.append((time.perf_counter() - t0) * 1e3)
    host_p50, host_p99 = percentile(host[5:], 50), percentile(host[5:], 99)

    # Resumable DDIM-10 solve, one step per advance call (host pointers, engine.h:321-366).
    out1 = np.empty((spec.horizon, spec.action_dim), np.float32)
    begins, advances, solves = [], [], []
    for i in range(25):
        t0 = time.perf_counter()
        eng.diffusion_begin(cond[0], noise[0], steps=steps_ddim)
        t1 = time.perf_counter()
        per = []
        for _ in range(steps_ddim):
            ta = time.perf_counter()
            eng.diffusion_advance(out1, 1)
            per.append((time.perf_counter() - ta) * 1e3)
        if i >= 5:
            begins.append((t1 - t0) * 1e3)
            advances.extend(per)
            solves.append((time.perf_counter() - t0) * 1e3)
    resumable = {"begin_p50_ms": round(percentile(begins, 50), 4),
                 "advance_1step_p50_ms": round(percentile(advances, 50), 4),
                 "advance_1step_p99_ms": round(percentile(advances, 99), 4),
                 "solve_p50_ms": round(percentile(solves, 50), 4),
                 "definition": "host-to-host: begin uploads condition/noise; each advance runs "
                               "one DDIM step and copies the current action back"}
    print(f"[bench] resumable DDIM-10: begin {resumable['begin_p50_ms']:.3f} ms, advance(1) "
          f"{resumable['advance_1step_p50_ms']:.3f} ms", file=sys.stderr, flush=True)

    # The timed path's own output against the oracle (parity is tested in full by tests/).
    action = d_out.cpu().numpy()
    b1_err = oracle_check(path, cond, noise, action, steps_ddim, [0]) if not args.no_cpu else None

    # Large batch.
    large = None
    B = args.large_batch
    if B > 0:
        cb, nb = ck.inputs(spec, batch=B)
        d_cb = torch.from_numpy(cb).to(dev)
        d_nb = torch.from_numpy(nb).to(dev)
        d_ob = torch.empty((B, spec.horizon, spec.action_dim), dtype=torch.float32, device=dev)
        eng.prepare(0, B, steps_ddim, 0)
        tick(B, d_cb, d_nb, d_ob)
        torch.cuda.synchronize()
        bl, bd = [], []
        for _ in range(args.large_steps):
            t0 = time.perf_counter()
            tick(B, d_cb, d_nb, d_ob)
            bl.append((time.perf_counter() - t0) * 1e3)
            bd.append(eng.last_device_ms)
        bp50 = percentile(bl, 50)
        flops_tick = nfe_flops * B * steps_ddim
        out_b = d_ob.cpu().numpy()
        sub = sorted({0, 1, 15, 16, 63, 64, 127, 128, 129, 191, 192, 200, 239, 240, B - 2, B - 1})
        sub = [i for i in sub if i < B]
        err_b = oracle_check(path, cb, nb, out_b, steps_ddim, sub) if not args.no_cpu else None
        large = {
            "batch": B, "p50_ms": bp50, "device_p50_ms": percentile(bd, 50),
            "actions_per_sec": B * spec.horizon / (bp50 / 1e3),
            "chunks_per_sec": B / (bp50 / 1e3),
            "tflops": flops_tick / (percentile(bd, 50) / 1e3) / 1e12,
            "mfma_peak_tflops": FP32_MFMA_PEAK_TFLOPS,
            "finite": bool(np.all(np.isfinite(out_b))),
            "max_abs_err_vs_oracle": err_b,
            "oracle_samples": sub,
        }
        large["frac_of_fp32_mfma_peak"] = large["tflops"] / FP32_MFMA_PEAK_TFLOPS
        print(f"[bench] B={B} DDIM-10 tick p50 {bp50:.2f} ms", file=sys.stderr, flush=True)
        bd_large = conv_breakdown(eng, batch=B, iters=5)
        for r in bd_large:
            print(f"[bench] B={B} {r['shape']:34s} x{r['launches_per_nfe']}  {r['us_per_launch']:9.1f} us"
                  f"  {r.get('tflops', 0):6.1f} TFLOP/s  {r['us_per_nfe']:9.1f} us/NFE",
                  file=sys.stderr, flush=True)
        large["conv_breakdown"] = [{k: v for k, v in r.items() if k != "indices"} for r in bd_large]

        # The same batch with F32 weights and inputs each split into two BF16 terms on the BF16
        # matrix cores (opt-in FLOWEDGE_MFMA_F32_SPLIT=1 at load: Wh Xh + Wh Xl + Wl Xh per
        # product, the Wl Xl term of ~2^-16 relative dropped, fp32 accumulation).  Reported beside
        # the exact-F32 line above, with its own error against the oracle on the same rows.
        if not args.no_split:
            os.environ["FLOWEDGE_MFMA_F32_SPLIT"] = "1"
            try:
                eng_s = flowedge_amd.Engine(path)
            finally:
                del os.environ["FLOWEDGE_MFMA_F32_SPLIT"]
            eng_s.prepare(0, B, steps_ddim, 0)

            def tick_s():
                eng_s.sample_device(0, d_cb.data_ptr(), d_nb.data_ptr(), B, steps_ddim, 0, 0,
                                    d_ob.data_ptr())

            tick_s()
            torch.cuda.synchronize()
            sl, sd = [], []
            for _ in range(args.large_steps):
                t0 = time.perf_counter()
                tick_s()
                sl.append((time.perf_counter() - t0) * 1e3)
                sd.append(eng_s.last_device_ms)
            sp50 = percentile(sl, 50)
            out_s = d_ob.cpu().numpy()
            err_s = oracle_check(path, cb, nb, out_s, steps_ddim, sub) if not args.no_cpu else None
            useful = flops_tick / (percentile(sd, 50) / 1e3) / 1e12
            large["f32_split_bf16_mfma"] = {
                "p50_ms": sp50, "device_p50_ms": percentile(sd, 50),
                "actions_per_sec": B * spec.horizon / (sp50 / 1e3),
                "useful_tflops": useful,
                "bf16_mfma_frac": 3 * useful / BF16_MFMA_PEAK_TFLOPS,
                "finite": bool(np.all(np.isfinite(out_s))),
                "max_abs_err_vs_oracle": err_s,
                "oracle_samples": sub,
                "arithmetic": "F32 weights and inputs split into BF16 hi + lo terms, three BF16 "
                              "MFMA products (hi*hi + hi*lo + lo*hi), fp32 accumulation; opt-in "
                              "FLOWEDGE_MFMA_F32_SPLIT=1",
            }
            print(f"[bench] B={B} DDIM-10 tick p50 {sp50:.2f} ms on BF16 matrix cores with split "
                  f"F32 operands (max err {err_s})", file=sys.stderr, flush=True)
            eng_s.close()

    breakdown = conv_breakdown(eng, batch=1)
    for r in breakdown:
        print(f"[bench] {r['shape']:34s} x{r['launches_per_nfe']}  {r['us_per_launch']:8.2f} us"
              f"  {r['gbs']:7.1f} GB/s  {r['us_per_nfe']:8.1f} us/NFE", file=sys.stderr, flush=True)
    roof = dominant_roofline(eng, args.roofline_iters)

    achieved = tick_bytes / (dev_p50 / 1e3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(p50, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(p50 / 810.0, 6),
        "vs_baseline_note": "value / 810 ms (reference native 10-step DDIM p50, caller thread, "
                            "docs/performance.md:59-64); lower is better",
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "LeRobot diffusion_pusht-size ConditionalUnet1D, DDIM 10 steps, batch 1",
            "dims": list(spec.dims), "horizon": spec.horizon, "action_dim": spec.action_dim,
            "cond_dim": spec.cond_dim, "kernel": spec.kernel, "groups": spec.groups,
            "train_timesteps": spec.train_timesteps, "batch": 1, "inference_steps": steps_ddim,
            "inputs": "device-resident (fe_engine_sample_device)",
        },
        "p99_ms": round(percentile(lat, 99), 4),
        "device_p50_ms": round(dev_p50, 4),
        "host_to_host_p50_ms": round(host_p50, 4),
        "host_to_host_p99_ms": round(host_p99, 4),
        "actions_per_sec_b1": round(spec.horizon / (p50 / 1e3), 1),
        "actions_per_sec_definition": "batch * horizon / p50 tick seconds",
        "resumable_b1": resumable,
        "large_batch": large,
        "roofline": roof,
        "tick_roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "kernel": "sampling tick (one hipGraph replay: 10 U-Net evaluations + updates)",
            "algorithmic_bytes_per_launch": tick_bytes,
        },
        "conv_breakdown_b1": [{k: v for k, v in r.items() if k != "indices"} for r in breakdown],
        "finite": bool(np.all(np.isfinite(action))),
        "max_abs_err_vs_oracle_b1": b1_err,
        "value_definition": "device-resident inputs (condition and noise already in HBM), one "
                            "fe_engine_sample_device call per tick, host-timed; the host-to-host "
                            "tick through fe_engine_sample_diffusion (PCIe included) is "
                            "host_to_host_p50_ms",
    }
    if not args.no_extra:
        result["other_configs"] = extra_configs(check=not args.no_cpu)
        result["observation_encoder"] = encoder_timing(2)
    if not args.no_cpu:
        cpu = cpu_baseline(path, spec, args.cpu_budget)
        result["cpu_baseline"] = {
            "value": round(cpu["threads1"]["p50_ms"], 2),
            "unit": "ms",
            "cores": 1,
            "kind": "port",
            "sample": f"{cpu['threads1']['ticks']} full B=1 DDIM-10 ticks, caller thread only",
            "threads8": {"value": round(cpu["threads8"]["p50_ms"], 2), "cores": 8,
                         "ticks": cpu["threads8"]["ticks"]},
            "all_cores": {"value": round(cpu["all_cores"]["p50_ms"], 2),
                          "cores": cpu["all_cores"]["cores"], "ticks": cpu["all_cores"]["ticks"]},
            "b256_extrapolated": {
                "threads1_ms": round(cpu["b256_threads1"]["ms"], 1),
                "all_cores_ms": round(cpu["b256_all_cores"]["ms"], 1),
                "cores": cpu["b256_all_cores"]["cores"],
                "sample": cpu["b256_all_cores"]["sample"] + "; threads1: "
                          + cpu["b256_threads1"]["sample"]},
            "cpu": cpu["cpu"],
            "note": "all_cores uses the host's CPU share for one GPU (16 cores), not its "
                    "hardware_concurrency; the oracle is this repository's AVX2 restatement of "
                    "the reference CPU path (the reference itself does not build with this "
                    "image's libstdc++)",
        }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
