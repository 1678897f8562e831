#!/usr/bin/env python3
"""Benchmark of the LeanKV decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads:
  gemv    config 1: TEAL sparse GEMV W[4096,14336], x ~Laplace(0,.05), 40 % sparse
  mlp     config 2: fused gate/up SwiGLU [14336,4096] + sparse down [4096,14336]
  quant   config 3: TurboQuant 3-bit quantize of K,V [8,4096,128] (fp32 MFMA rotation)
  attn    config 4: packed-KV decode attention, B=16, 32/8 heads, ctx 4096 + 64 hot
Every workload rotates >= 3 independent buffer sets (> 512 MB) so the 256 MB
Infinity Cache cannot serve repeated launches.  A "step" is one launch of the
workload's kernel(s) over one buffer set.  Timing: W untimed steps, then K timed
steps bracketed by torch.cuda.synchronize(); the dominant kernel's average
duration comes from HIP events recorded around each launch on the stream the
kernels run on (torch's current stream).  Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, AMD spec
MFMA_F32_PEAK_TFLOPS = 157.3


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="gemv", choices=["gemv", "mlp", "quant", "attn"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sets", type=int, default=5, help="independent buffer sets rotated per step")
    return ap.parse_args()


def _timed_loop(launch, nsets, steps, warmup, torch):
    """Run launch(i % nsets); return (wall ms/step, mean kernel ms from per-launch events)."""
    for i in range(warmup):
        launch(i % nsets)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        evs[i][0].record()
        launch(i % nsets)
        evs[i][1].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    durs = [a.elapsed_time(b) for a, b in evs]
    return wall, statistics.mean(durs), statistics.median(durs)


def _cpu_info():
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cores, model


# ------------------------------------------------------------------ config 1
def bench_gemv(args, torch):
    from leankv_amd import kernels

    dev = torch.device("cuda:0")
    N, Z = 4096, 14336
    sets = []
    for s in range(args.sets):
        g = torch.Generator(device=dev).manual_seed(s)
        W = (torch.randn(N, Z, generator=g, device=dev) * 0.02).half()
        Wc = W.t().contiguous().t()
        del W
        torch.manual_seed(s)
        x = torch.distributions.Laplace(0.0, 0.05).sample((Z,)).half().to(dev)
        t = torch.kthvalue(x.float().abs().cpu(), int(0.4 * Z)).values.item()
        surv = int((x.float().abs() > t).sum())
        sets.append((x, Wc, t, surv, torch.empty(N, dtype=torch.float16, device=dev)))
    def launch(i):
        x, Wc, t, _, y = sets[i]
        kernels.sparse_gemv_out(x, Wc, t, y)
    wall, kmean, kmed = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    surv = statistics.mean(s[3] for s in sets)
    alg_bytes = surv * N * 2 + Z * 2 + N * 2
    achieved = alg_bytes / (kmean * 1e-3) / 1e9
    res = {
        "metric": "sparse GEMV HBM GB/s (W[4096,14336] fp16, 40% sparse x)",
        "value": round(achieved, 1),
        "unit": "GB/s",
        "ms_per_step": round(wall, 5),
        "higher_is_better": True,
        "dtype": "f16 (fp32 accumulate)",
        "config": {"workload": "config1_sparse_gemv", "N": N, "Z": Z, "sparsity": 0.4,
                   "buffer_sets": len(sets), "working_set_MB": round(len(sets) * N * Z * 2 / 1e6)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "sparse_gemv_kernel", "kernel_us_mean": round(kmean * 1e3, 3),
                     "kernel_us_median": round(kmed * 1e3, 3), "alg_bytes_per_launch": int(alg_bytes)},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_gemv(torch, sets[0], N, Z)
    return res


def cpu_gemv(torch, s, N, Z):
    """Reference semantics on the host: x * (|x| > t) then F.linear (fp32)."""
    x, Wc, t, _, _ = s
    W = Wc.float().cpu().contiguous()
    xx = x.float().cpu()
    cores, model = _cpu_info()
    torch.set_num_threads(cores)
    f = lambda: torch.nn.functional.linear(xx * (xx.abs() > t), W)
    for _ in range(3):
        f()
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 10.0 or reps < 10:
        f()
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    surv = int((xx.abs() > t).sum())
    gbs = (surv * N * 2 + Z * 2 + N * 2) / dt / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s (same algorithmic bytes)", "cores": cores,
            "kind": "port", "sample": "config 1 GEMV, %d reps in ~10 s, torch fp32 on %s" % (reps, model),
            "ms_per_call": round(dt * 1e3, 3)}


def main():
    args = _parse()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (single-GPU decode hot path); "
              "--gpus %d is not supported" % args.gpus, file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    fn = {"gemv": bench_gemv}[args.workload]
    res = fn(args, torch)
    out = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup}
    out.update(res)
    out.setdefault("scaling", "weak")
    out.setdefault("vs_baseline", None)
    out.setdefault("data", "synthetic (seeded)")
    print(json.dumps(out))


if __name__ == "__main__":
    main()
