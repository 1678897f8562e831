#!/usr/bin/env python3
"""Benchmark of the LeanKV decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads (the benchmark configurations 1-5 of the decode hot path):
  decode  config 5 (default): random-init fp16 Mistral-7B-v0.3-shaped decoder, 4096-token
          random prompt, per-projection TEAL sparsity ~U[0.3,0.5] (thresholds from a seeded
          calibration pass at the decode context: quantiles over the last 256 positions of a
          4096-token prompt), 3-bit TurboQuant KV (64-token fp16 window), greedy B=1 decode of
          warmup+steps = 128 tokens through the graph-captured LeanKV engine.  Beside it on the
          same prompt: two dense fp16 baselines with an fp16 KV cache, both graph-captured --
          the same fused step on this library's kernels with every threshold 0 (own_kernels;
          speedup_vs_dense is taken against the faster of the two) and torch F.linear + SDPA --
          and HF model.generate tok/s, prefill included, dense and LeanKV (the reference's
          method, scripts/benchmark.py:68-99).  step_roofline counts the weight rows above
          threshold on the timed tokens (replayed through the HF path, whose activations equal
          the engine's) and reports bytes per token over ms_per_step.
          value = decode tok/s of the LeanKV engine (prefill excluded).
  dense   the dense fp16 baseline of config 5 alone: this library's decode step with every
          threshold 0 and an fp16 KV cache in 16-token pages (OwnDenseEngine), graph-captured;
          value = tok/s, step_roofline = dense bytes per token / ms_per_step (for profiling it)
  gemv    config 1: TEAL sparse GEMV W[4096,14336], x ~Laplace(0,.05), 40 % sparse
  mlp     config 2: fused gate/up SwiGLU [14336,4096] + sparse down [4096,14336]
  quant   config 3: TurboQuant 3-bit quantize of K,V [8,4096,128] (fp32 MFMA rotation)
  attn    config 4: packed-KV decode attention, B=16, 32/8 heads, ctx 4096 + 64 hot
  prefill causal prefill attention of one config-5 layer over its packed cache (4096-token
          prompt, 32/8 heads; MFMA-bound, so 3 buffer sets), beside the reference path
          (dequantize + torch SDPA) on the same GPU
  batched B=8 decode rows through one TEAL-sparse projection (config-1 shape), beside 8 single-row
          GEMV calls and torch's dense GEMM
  paged   batch decode attention on the paged fp16 pool (B=16, 4096 tokens, 16-token pages),
          beside torch SDPA on the same K/V held dense
  tqpaged config 4 through a paged 3-bit cache (4096 cold tokens per sequence in 16-token pages
          scattered over the pool), beside the dense packed kernel on the same codes
  prod    TurboQuantProd 3-bit (2-bit MSE + 1-bit QJL) quantize of the config-3 K,V fp16 [8,4096,128],
          fp32-MFMA bound (three 128x128 products per vector); dequantize and the reference's torch
          formulation on the same GPU timed beside it
  copy    a 512 MiB device copy: the known-size reference for scaling PMC byte counters
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
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode", choices=["decode", "dense", "gemv", "mlp", "quant", "attn",
                                                                    "prefill", "batched", "paged", "tqpaged", "prod",
                                                                    "copy", "generate"])
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=32, help="decoder layers (config 5 uses 32)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-dense", action="store_true", help="skip the dense fp16 comparison run")
    ap.add_argument("--no-roofline", action="store_true", help="skip the config-1 GEMV roofline measurement")
    ap.add_argument("--sets", type=int, default=5, help="independent buffer sets rotated per step")
    ap.add_argument("--cold", type=int, default=4096, help="--workload attn: cold tokens per sequence (config 4: 4096)")
    ap.add_argument("--phases", action="store_true",
                    help="--workload attn / decode: add per-block phase times of the attention kernels; needs the "
                         "instrumented build (python -m leankv_amd.build --stamps) loaded through "
                         "LKV_LIBRARY=leankv_amd/libleankv_amd_stamps.so")
    ap.add_argument("--batches", default="4,16",
                    help="--workload generate: batch sizes, comma-separated (the value is the largest one's)")
    ap.add_argument("--no-hf-forward", action="store_true",
                    help="--workload generate: skip the comparison runs on the patched HF forward")
    ap.add_argument("--bits", type=int, default=3, choices=(1, 2, 3, 4),
                    help="--workload attn / decode: code width of the packed cache (configs 4 and 5: 3; the "
                         "reference sweeps 2.5-4 bits, configs/mistral7b.yaml)")
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


def _kernel_time(launch, nsets, steps, warmup, torch, batch=10):
    """Average duration of one launch: HIP events around batches of `batch` back-to-back launches on the
    launching stream (a lone launch between two events also times its dispatch latency).  For a kernel of
    ~13 us the host must issue a launch in less than that or the events time the host instead: the GEMV
    rooflines launch through a pre-bound C entry point (_fast_partials) for that reason."""
    for i in range(warmup):
        launch(i % nsets)
    torch.cuda.synchronize()
    nb = max(1, steps // batch)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nb)]
    for j, (a, b) in enumerate(evs):
        a.record()
        for i in range(batch):
            launch((j * batch + i) % nsets)
        b.record()
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) / batch for a, b in evs]
    return statistics.mean(per), statistics.median(per)


def _bound(name, *args):
    """A launch closure over one C entry point with its arguments converted once (ints, floats, pointers):
    the per-launch host cost is one ctypes call, so back-to-back launches of a ~13 us kernel are not spaced
    by Python-side argument checks.  The caller has made the same call through the checked wrapper first."""
    from leankv_amd import _lib
    fn = getattr(_lib.load(), name)

    def call(_i=None):
        rc = fn(*args)
        if rc != 0:
            raise _lib.LeanKVError("%s failed: %s" % (name, _lib.last_error()))
    return call


def _cpu_info():
    """(threads for the CPU baseline, CPU model): the cores this process may run on (affinity mask),
    capped by OMP_NUM_THREADS when the machine sets a CPU share that way."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        cores = min(cores, int(omp))
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
    from leankv_amd._lib import workspaces

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
    wall, eager, _ = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    lib = kernels._lib_handle()
    ws = workspaces.get(dev, "gemv", lib.lkv_sparse_gemv_workspace_bytes(N, Z))
    st = torch.cuda.current_stream().cuda_stream
    fast = [_bound("lkv_sparse_gemv", x.data_ptr(), Wc.data_ptr(), float(t), N, Z, y.data_ptr(), ws.data_ptr(),
                   ws.numel(), st) for x, Wc, t, _, y in sets]
    omean, _ = _kernel_time(lambda i: fast[i](), len(sets), args.steps, args.warmup, torch)
    surv = statistics.mean(s[3] for s in sets)
    alg_bytes = surv * N * 2 + Z * 2 + N * 2
    roof = _roofline_partials(torch, [(s[0], s[1], s[2], None, 0.0) for s in sets], N, Z, alg_bytes,
                              args.steps, args.warmup, "sparse_gemv_kernel (config 1 split-K pass)")
    res = {
        "metric": "sparse GEMV HBM GB/s (W[4096,14336] fp16, 40% sparse x)",
        "value": round(alg_bytes / (omean * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "ms_per_step": round(wall, 5),
        "op_us_back_to_back": round(omean * 1e3, 3),
        "op_us_eager_call": round(eager * 1e3, 3),
        "higher_is_better": True,
        "dtype": "f16 (fp32 accumulate)",
        "config": {"workload": "config1_sparse_gemv", "N": N, "Z": Z, "sparsity": 0.4,
                   "buffer_sets": len(sets), "working_set_MB": round(len(sets) * N * Z * 2 / 1e6),
                   "what": "value: whole op (split-K pass + chunk reduction) per call, calls issued back to "
                           "back through the C entry point; op_us_eager_call: one call through the Python "
                           "wrapper between two events; roofline: split-K pass"},
        "roofline": roof,
    }
    if args.phases:
        res["phases"] = _phases(torch, lambda: launch(0))
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_gemv(torch, sets[0], N, Z)
    return res


TRAFFIC_SOURCE = ("profiles/traffic.json: committed rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE means of this kernel at "
                  "this shape (separate counter runs, scaled by a device copy's factors), not measured in this run")


def _traffic(kernel_key):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC summary (None if absent)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel_key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def _roofline_partials(torch, sets, N, Z, alg_bytes, steps, warmup, name, key=None):
    """Average duration of the split-K GEMV kernel alone, from HIP events around each launch.

    sets: (x, w_gate, t_gate, w_up or None, t_up); one kernel per launch."""
    from leankv_amd import kernels

    outs = [kernels.sparse_gemv_partials(x, wg, tg, wu, tu) for x, wg, tg, wu, tu in sets]
    st = torch.cuda.current_stream().cuda_stream
    fast = [_bound("lkv_sparse_gemv_partials", x.data_ptr(), wg.data_ptr(), None if wu is None else wu.data_ptr(),
                   float(tg), float(tu), N, Z, o.data_ptr(), o.numel() * 4, st)
            for (x, wg, tg, wu, tu), o in zip(sets, outs)]

    def launch(i):
        fast[i]()
    kmean, kmed = _kernel_time(launch, len(sets), steps, warmup, torch)
    _, single, _ = _timed_loop(launch, len(sets), steps // 2, 0, torch)
    achieved = alg_bytes / (kmean * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _traffic(key or "gemv_config1"), "traffic_source": TRAFFIC_SOURCE,
            "kernel": name, "kernel_us_mean": round(kmean * 1e3, 3), "kernel_us_median": round(kmed * 1e3, 3),
            "kernel_us_single_launch_events": round(single * 1e3, 3), "alg_bytes_per_launch": int(alg_bytes)}


def roofline_gateup(args, torch):
    """The dominant decode kernel: fused TEAL gate/up GEMV at the Mistral-7B shape (config 2 inputs).

    Wg, Wu [14336, 4096] ~N(0,.02), x[4096] ~N(0,1), both thresholds at the 40 % quantile of |x|;
    3 buffer sets (705 MB) rotate so the Infinity Cache cannot serve them."""
    dev = torch.device("cuda:0")
    N, Z = 14336, 4096
    sets, surv = [], []
    for s in range(3):
        g = torch.Generator(device=dev).manual_seed(100 + s)
        wg = (torch.randn(N, Z, generator=g, device=dev) * 0.02).half().t().contiguous().t()
        wu = (torch.randn(N, Z, generator=g, device=dev) * 0.02).half().t().contiguous().t()
        x = torch.randn(Z, generator=g, device=dev).half()
        t = torch.kthvalue(x.float().abs().cpu(), int(0.4 * Z)).values.item()
        surv.append(int((x.float().abs() > t).sum()))
        sets.append((x, wg, t, wu, t))
    alg = 2 * statistics.mean(surv) * N * 2 + Z * 2 + 2 * N * 2
    r = _roofline_partials(torch, sets, N, Z, alg, 200, 20, "sparse_gemv_kernel (fused gate/up, config-5 shape)",
                           key="gemv_gateup_config5")
    del sets
    torch.cuda.empty_cache()
    return r


def cpu_decode(torch, model, thresholds, prompt_len, budget_s=20.0, bits=3):
    """The reference's decode path on the host (oracle restatement, torch fp32), bounded sample.

    One decoder layer of the same random model with its TEAL thresholds and a TurboQuant cache
    holding prompt_len tokens (random fp16 K/V: the cost does not depend on the values), decoding
    token by token for ~budget_s seconds; tok/s = 1 / (32 x layer time + embed/norm/lm_head time)."""
    import copy

    from oracle import turboquant as oq
    from oracle.model import RefModel

    cores, cpu = _cpu_info()
    torch.set_num_threads(cores)
    cfg = copy.deepcopy(model.config)
    cfg.num_hidden_layers = 1
    keep = ("model.embed_tokens.", "model.layers.0.", "model.norm.", "lm_head.")
    state = {k: v.detach().float().cpu() for k, v in model.state_dict().items() if k.startswith(keep)}
    ref = RefModel(state, cfg, {0: thresholds[0]}, bits=bits, acc_dtype=torch.float32)
    g = torch.Generator().manual_seed(0)
    Hkv, D = cfg.num_key_value_heads, 128
    ref.caches[0].update(torch.randn(1, Hkv, prompt_len, D, generator=g).half(),
                         torch.randn(1, Hkv, prompt_len, D, generator=g).half())
    ref.pos = prompt_len
    tok = torch.tensor([1])
    ref.forward(tok)  # warm-up step
    ref.t_layers = ref.t_head = 0.0
    n, t0 = 0, time.perf_counter()
    while n < 3 or time.perf_counter() - t0 < budget_s:
        ref.forward(tok)
        n += 1
    layer_s, head_s = ref.t_layers / n, ref.t_head / n
    L = model.config.num_hidden_layers
    return {"value": round(1.0 / (L * layer_s + head_s), 4), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": "%d decode steps of 1 of %d layers at context %d (TEAL thresholds, %d-bit TurboQuant cache "
                      "re-dequantized every step as the reference does), oracle torch fp32 on %s; "
                      "per token = %d x %.1f ms/layer + %.1f ms embed/norm/lm_head"
                      % (n, L, prompt_len, bits, cpu, L, layer_s * 1e3, head_s * 1e3)}


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


# ------------------------------------------------------------------ config 2
def bench_mlp(args, torch):
    """Config 2: fused sparse gate/up SwiGLU (x ~N(0,1) at 40 %) then sparse down at 40 % of |h|.

    value: algorithmic bytes of both ops / their combined time per call; roofline: the gate/up
    split-K pass alone (the decode step's dominant kernel)."""
    from leankv_amd import kernels
    from leankv_amd._lib import workspaces

    dev = torch.device("cuda:0")
    H, F = 4096, 14336
    sets, alg = [], []
    for s in range(args.sets if args.sets <= 3 else 3):
        g = torch.Generator(device=dev).manual_seed(200 + s)
        wg = (torch.randn(F, H, generator=g, device=dev) * 0.02).half().t().contiguous().t()
        wu = (torch.randn(F, H, generator=g, device=dev) * 0.02).half().t().contiguous().t()
        wd = (torch.randn(H, F, generator=g, device=dev) * 0.02).half().t().contiguous().t()
        x = torch.randn(H, generator=g, device=dev).half()
        tx = torch.kthvalue(x.float().abs().cpu(), int(0.4 * H)).values.item()
        h = kernels.sparse_gateup_swiglu(x, wg, wu, tx, tx)
        th = torch.kthvalue(h.float().abs().cpu(), int(0.4 * F)).values.item()
        sx = int((x.float().abs() > tx).sum())
        sh = int((h.float().abs() > th).sum())
        alg.append(2 * sx * F * 2 + sh * H * 2 + H * 2 + 2 * F * 2 + H * 2)
        sets.append((x, wg, wu, wd, tx, th, h, torch.empty(H, dtype=torch.float16, device=dev)))

    def launch(i):
        x, wg, wu, wd, tx, th, h, y = sets[i]
        kernels.sparse_gateup_swiglu_out(x, wg, wu, tx, tx, h)
        kernels.sparse_gemv_out(h, wd, th, y)
    wall, eager, _ = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    lib = kernels._lib_handle()
    st = torch.cuda.current_stream().cuda_stream
    wgu = workspaces.get(dev, "gateup", lib.lkv_sparse_gateup_workspace_bytes(F, H))
    wdn = workspaces.get(dev, "gemv", lib.lkv_sparse_gemv_workspace_bytes(H, F))
    fast = []
    for x, wg, wu, wd, tx, th, h, y in sets:
        f1 = _bound("lkv_sparse_gateup_swiglu", x.data_ptr(), wg.data_ptr(), wu.data_ptr(), float(tx), float(tx), F, H,
                    h.data_ptr(), wgu.data_ptr(), wgu.numel(), st)
        f2 = _bound("lkv_sparse_gemv", h.data_ptr(), wd.data_ptr(), float(th), H, F, y.data_ptr(), wdn.data_ptr(),
                    wdn.numel(), st)
        fast.append((f1, f2))

    def fast_launch(i):
        fast[i][0]()
        fast[i][1]()
    omean, _ = _kernel_time(fast_launch, len(sets), args.steps, args.warmup, torch)
    a = statistics.mean(alg)
    gu_alg = statistics.mean(2 * int((x.float().abs() > tx).sum()) * F * 2 + H * 2 + 2 * F * 2
                             for x, _, _, _, tx, _, _, _ in sets)
    roof = _roofline_partials(torch, [(x, wg, tx, wu, tx) for x, wg, wu, _, tx, _, _, _ in sets], F, H, gu_alg,
                              args.steps, args.warmup, "sparse_gemv_kernel (fused gate/up split-K pass)",
                              key="gemv_gateup_config5")
    return {
        "metric": "fused sparse MLP HBM GB/s (gate/up [14336,4096] + down [4096,14336], 40% sparse)",
        "value": round(a / (omean * 1e-3) / 1e9, 1), "unit": "GB/s", "ms_per_step": round(wall, 5),
        "op_us_back_to_back": round(omean * 1e3, 3), "op_us_eager_call": round(eager * 1e3, 3),
        "higher_is_better": True, "dtype": "f16 (fp32 accumulate)",
        "config": {"workload": "config2_fused_mlp", "hidden": H, "ffn": F, "sparsity": 0.4,
                   "buffer_sets": len(sets), "alg_bytes_per_call": int(a),
                   "what": "value: gate/up + down per call, calls issued back to back through the C entry "
                           "points; op_us_eager_call: one call through the Python wrappers between two events"},
        "roofline": roof,
    }


def bench_copy(args, torch):
    """A plain device copy of known size (512 MiB read + 512 MiB written per step): the reference point
    for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes."""
    dev = torch.device("cuda:0")
    n = 512 << 20
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    wall, kmean, _ = _timed_loop(lambda i: b.copy_(a), 1, args.steps, args.warmup, torch)
    return {"metric": "device copy GB/s (read + write)", "value": round(2 * n / (kmean * 1e-3) / 1e9, 1),
            "unit": "GB/s", "ms_per_step": round(wall, 5), "higher_is_better": True, "dtype": "u8",
            "config": {"workload": "copy_512MiB", "bytes_read": n, "bytes_written": n}}


# ------------------------------------------------------------------ config 3
def bench_quant(args, torch):
    """Config 3: TurboQuant 3-bit quantize of K and V fp16 [8, 4096, 128] (4 channels x10), Pi seeds 42/43.

    One step = quantize K (PiK) + quantize V (PiV): norm, normalise, fp32-MFMA rotation, bucketing and
    nibble packing in one kernel each; 32 rotating K/V sets (537 MB)."""
    from leankv_amd import kernels
    from leankv_amd.turboquant.codebook import get_codebook_tensors
    from leankv_amd.turboquant.rotation import generate_rotation_matrix

    dev = torch.device("cuda:0")
    H, T, D = 8, 4096, 128
    _, bnd = get_codebook_tensors(D, 3, dev, torch.float32)
    bounds = bnd[1:-1].contiguous()
    PiK = generate_rotation_matrix(D, dev, torch.float32, 42)
    PiV = generate_rotation_matrix(D, dev, torch.float32, 43)
    sets = []
    for s in range(32):
        g = torch.Generator(device=dev).manual_seed(300 + s)
        kv = torch.randn(2, H, T, D, generator=g, device=dev)
        kv[..., [0, 31, 64, 127]] *= 10
        sets.append(kv.half())

    def launch(i):
        kernels.tq_quantize(sets[i][0], PiK, bounds, 3)
        kernels.tq_quantize(sets[i][1], PiV, bounds, 3)
    wall, omean, _ = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    kmean, kmed = _kernel_time(launch, len(sets), args.steps, args.warmup, torch)
    nvec = 2 * H * T
    alg_bytes = nvec * (D * 2 + 64 + 2)
    flops = nvec * 2 * D * D
    tflops = flops / (kmean * 1e-3) / 1e12
    return {
        "metric": "TurboQuant 3-bit quantize GB/s (K,V fp16 [8,4096,128])",
        "value": round(alg_bytes / (kmean * 1e-3) / 1e9, 1), "unit": "GB/s", "ms_per_step": round(wall, 5),
        "higher_is_better": True, "dtype": "fp32 rotation (fp16 in, 3-bit codes + fp16 norms out)",
        "config": {"workload": "config3_tq_quantize", "vectors": nvec, "alg_bytes_per_step": alg_bytes,
                   "rotation_flop_per_step": flops, "sets": len(sets)},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_F32_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "quantize_wave_kernel<3,true> (K and V launches)", "kernel_us_mean": round(kmean * 1e3, 3),
                     "kernel_us_median": round(kmed * 1e3, 3), "hbm_GBps": round(alg_bytes / (kmean * 1e-3) / 1e9, 1)},
    }


# ------------------------------------------------------------------ TurboQuantProd (QJL)
PROD_Q_BYTES = 128 * 2 + 32 + 2 + 16 + 4   # fp16 vector in; 2-bit codes, fp16 norm, signs, fp32 rnorm out
PROD_DQ_BYTES = 32 + 2 + 16 + 4 + 128 * 4  # codes, norm, signs, rnorm in; fp32 vector out
PROD_Q_FLOP = 3 * 2 * 128 * 128            # x Pi^T, y Pi, r S^T
PROD_DQ_FLOP = 2 * 2 * 128 * 128           # y Pi, s S


def bench_prod(args, torch):
    """TurboQuantProd at 3 bits (2-bit MSE codes + 1-bit QJL signs + residual norm) of the config-3 K and V
    fp16 [8, 4096, 128] (4 channels x10), seeds 42 (K) / 43 (V), S from seed + 1000.  One step = quantize K
    and V, one fused kernel each (three fp32-MFMA 128x128 products per vector); dequantize (two products)
    is timed beside it, and the reference's torch formulation of quantize on the same GPU."""
    from leankv_amd import _lib
    from leankv_amd.turboquant.quantizer import TurboQuantProd

    dev = torch.device("cuda:0")
    H, T, D = 8, 4096, 128
    tqs = (TurboQuantProd(D, 3, device=dev, seed=42), TurboQuantProd(D, 3, device=dev, seed=43))
    lib = _lib.load()
    st = _lib.stream_handle(dev)
    M = H * T
    sets = []
    for s in range(16):
        g = torch.Generator(device=dev).manual_seed(500 + s)
        kv = torch.randn(2, H, T, D, generator=g, device=dev)
        kv[..., [0, 31, 64, 127]] *= 10
        kv = kv.half()
        outs = []
        for h in range(2):
            tq = tqs[h]
            q = tq.quantize(kv[h])
            outs.append((kv[h], q, torch.empty(H, T, D, device=dev)))
        sets.append(outs)
    ptr = _lib.ptr

    def quant(i):  # the C ABI straight, so that host overhead cannot hide between launches
        for h in range(2):
            x, q, _ = sets[i][h]
            m = tqs[h].mse_quantizer
            lib.lkv_tq_prod_quantize(ptr(x), 1, M, ptr(m.Pi), ptr(m.decision_boundaries), ptr(m.centroids),
                                     ptr(tqs[h].S), 2, ptr(q.mse_indices), ptr(q.norms), ptr(q.qjl_signs),
                                     ptr(q.residual_norms), st)

    def dequant(i):
        for h in range(2):
            _, q, out = sets[i][h]
            m = tqs[h].mse_quantizer
            lib.lkv_tq_prod_dequantize(ptr(q.mse_indices), ptr(q.norms), 1, ptr(q.qjl_signs), ptr(q.residual_norms),
                                       M, ptr(m.Pi), ptr(m.centroids), ptr(tqs[h].S), 2, tqs[h].qjl_scale, ptr(out),
                                       0, st)
    assert _lib.dtype_code(torch.float16) == 1 and _lib.dtype_code(torch.float32) == 0
    wall, _, _ = _timed_loop(quant, len(sets), args.steps, args.warmup, torch)
    kq, kq_med = _kernel_time(quant, len(sets), args.steps, args.warmup, torch)
    kd, _ = _kernel_time(dequant, len(sets), args.steps, args.warmup, torch)
    nvec = 2 * M
    q_bytes, q_flop = nvec * PROD_Q_BYTES, nvec * PROD_Q_FLOP
    d_bytes, d_flop = nvec * PROD_DQ_BYTES, nvec * PROD_DQ_FLOP
    tf = q_flop / (kq * 1e-3) / 1e12

    def torch_path(i):  # quantizer.py:119-129 + 206-222 as torch ops on the GPU
        for h in range(2):
            x = sets[i][h][0]
            m, S = tqs[h].mse_quantizer, tqs[h].S
            nrm = x.norm(dim=-1)
            y = torch.matmul((x / (nrm.unsqueeze(-1) + 1e-10)).float(), m.Pi.T)
            idx = torch.searchsorted(m.decision_boundaries, y.contiguous())
            packed = (idx.to(torch.uint8).reshape(H, T, 32, 4) << torch.tensor([0, 2, 4, 6], device=dev,
                      dtype=torch.uint8)).sum(-1, dtype=torch.uint8)
            xh = torch.matmul(m.centroids[idx], m.Pi) * nrm.unsqueeze(-1)
            r = x - xh
            rn = r.norm(dim=-1)
            bits = (torch.matmul(r.float(), S.T) > 0).to(torch.uint8).reshape(H, T, 16, 8)
            signs = (bits << torch.arange(8, device=dev, dtype=torch.uint8)).sum(-1, dtype=torch.uint8)
            del packed, rn, signs
    tt, _ = _kernel_time(torch_path, len(sets), min(args.steps, 50), 3, torch, batch=5)
    res = {
        "metric": "TurboQuantProd 3-bit quantize GB/s (K,V fp16 [8,4096,128])",
        "value": round(q_bytes / (kq * 1e-3) / 1e9, 1), "unit": "GB/s", "ms_per_step": round(wall, 5),
        "higher_is_better": True, "dtype": "fp32 MFMA (fp16 in; 2-bit codes, signs, norms out)",
        "config": {"workload": "tq_prod_quantize_config3", "vectors": nvec, "alg_bytes_per_step": q_bytes,
                   "flop_per_step": q_flop, "sets": len(sets),
                   "dequantize": {"kernel": "prod_dequantize_kernel<2,true,false>", "us_per_step": round(kd * 1e3, 2),
                                  "GBps": round(d_bytes / (kd * 1e-3) / 1e9, 1),
                                  "TFLOPs": round(d_flop / (kd * 1e-3) / 1e12, 2),
                                  "mfma_frac": round(d_flop / (kd * 1e-3) / 1e12 / MFMA_F32_PEAK_TFLOPS, 4)},
                   "reference_path_gpu": {"what": "the reference's quantize as torch ops on the same GPU",
                                          "us_per_step": round(tt * 1e3, 1), "speedup": round(tt / kq, 2)}},
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / MFMA_F32_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "prod_quantize_kernel<2,true> (K and V launches)",
                     "kernel_us_mean": round(kq * 1e3, 3), "kernel_us_median": round(kq_med * 1e3, 3),
                     "hbm_GBps": round(q_bytes / (kq * 1e-3) / 1e9, 1)},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = _cpu_prod(torch)
    return res


def _cpu_prod(torch):
    """The oracle's TurboQuantProd quantize (torch CPU ops, all host threads) on 8 heads' worth of K."""
    from oracle import turboquant as oq

    cores, model = _cpu_info()
    torch.set_num_threads(cores)
    Pi, S = oq.rotation_matrix(128, 42), oq.qjl_matrix(128, 1042)
    c, b = oq.codebook_tensors(2)
    g = torch.Generator().manual_seed(9)
    n, dt = 0, 0.0
    for _ in range(8):
        x = torch.randn(4096, 128, generator=g)
        x[:, [0, 31, 64, 127]] *= 10
        x = x.half()
        t = time.perf_counter()
        oq.prod_quantize(x, Pi, b, c, S, 2)
        dt += time.perf_counter() - t
        n += x.shape[0]
    return {"value": round(n * PROD_Q_BYTES / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": "oracle prod_quantize (torch CPU), 8 x 4096 fp16 vectors; %s" % model}


# ------------------------------------------------------------------ config 4
def bench_attn(args, torch):
    """Config 4: decode attention on the packed 3-bit cache, B=16, 32 query / 8 kv heads, 4096 cold tokens
    + a 64-token fp16 hot window, scale 1/sqrt(128).  The cache content is random 3-bit codes (both
    nibbles 0..7) and norms (the kernels' cost does not depend on it); 8 rotating cache sets (570 MB)."""
    from leankv_amd import kernels
    from leankv_amd.turboquant.codebook import get_codebook_tensors
    from leankv_amd.turboquant.rotation import generate_rotation_matrix

    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, cold, hot = 16, 32, 8, 128, args.cold, 64
    bits = args.bits
    rb = {1: 16, 2: 32}.get(bits, 64)  # packed code bytes per token
    L = cold + hot
    cent, _ = get_codebook_tensors(D, bits, dev, torch.float32)
    PiK = generate_rotation_matrix(D, dev, torch.float32, 42)
    PiV = generate_rotation_matrix(D, dev, torch.float32, 43)
    seq = torch.tensor([L], dtype=torch.int32, device=dev)
    sets = []
    for s in range(8):
        g = torch.Generator(device=dev).manual_seed(400 + s)
        mask = 0x77 if bits == 3 else 0xFF  # every code valid at its width
        kc = torch.randint(0, 256, (B, Hkv, cold, rb), generator=g, device=dev, dtype=torch.uint8) & mask
        vc = torch.randint(0, 256, (B, Hkv, cold, rb), generator=g, device=dev, dtype=torch.uint8) & mask
        kn = torch.rand(B, Hkv, cold, generator=g, device=dev) * 4 + 8
        vn = torch.rand(B, Hkv, cold, generator=g, device=dev) * 4 + 8
        kh = torch.randn(B, Hkv, hot, D, generator=g, device=dev).half()
        vh = torch.randn(B, Hkv, hot, D, generator=g, device=dev).half()
        q = torch.randn(B, Hq, D, generator=g, device=dev).half()
        sets.append((q, kc, kn, vc, vn, kh, vh, torch.empty_like(q)))
    ws = torch.empty(kernels.decode_attn_workspace_bytes(B, Hq, Hkv, L), dtype=torch.uint8, device=dev)

    def launch(i):
        q, kc, kn, vc, vn, kh, vh, out = sets[i]
        kernels.tq_decode_attn_out(q, kc, kn, vc, vn, kh, vh, PiK, PiV, cent, bits, seq, L, D ** -0.5, out, ws)
    wall, _, _ = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    kmean, kmed = _kernel_time(launch, len(sets), args.steps, args.warmup, torch)
    alg = B * Hkv * (cold * (rb + rb + 4 + 4) + hot * D * 2 * 2) + 2 * B * Hq * D * 2
    achieved = alg / (kmean * 1e-3) / 1e9
    phases = _phases(torch, lambda: launch(0)) if args.phases else None
    res = {
        "metric": "packed-KV decode attention HBM GB/s (B=16, 32/8 heads, 4096 cold + 64 hot)",
        "value": round(achieved, 1), "unit": "GB/s", "ms_per_step": round(wall, 5), "higher_is_better": True,
        "dtype": "%d-bit codes, fp16 MFMA scores/values, fp32 softmax" % bits,
        "config": {"workload": "config4_packed_attention", "batch": B, "heads": "32/8", "cold": cold, "hot": hot,
                   "bits": bits,
                   "alg_bytes_per_call": alg, "sets": len(sets)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _traffic("attn_config4"), "traffic_source": TRAFFIC_SOURCE,
                     "kernel": "tq_attn_split_kernel (q rotation in its prologue) + tq_attn_combine_kernel (one call)",
                     "kernel_us_mean": round(kmean * 1e3, 3), "kernel_us_median": round(kmed * 1e3, 3),
                     "alg_bytes_per_launch": alg},
    }
    if phases:
        res["phases"] = phases
    return res


def _split_phases(out, split, comb, st):
    """The attention split / combine part of _phases (times relative to the first split block's start)."""
    t0 = min(r[0] for r in split)
    out["split_blocks"] = len(split)
    out["split_start"] = st(r[0] - t0 for r in split)
    out["split_prologue"] = st(r[1] - r[0] for r in split)
    pro = [r for r in split if r[4] and r[5]]  # blocks with cold tokens: query ready, rotation done
    if pro:
        out["split_prologue_query_ready"] = st(r[4] - r[0] for r in pro)
        out["split_prologue_rotation"] = st(r[5] - r[4] for r in pro)
        out["split_prologue_after_rotation"] = st(r[1] - r[5] for r in pro)
    out["split_token_loop"] = st(r[2] - r[1] for r in split)
    out["split_merge_and_record"] = st(r[3] - r[2] for r in split)
    out["split_end"] = st(r[3] - t0 for r in split)
    if comb:
        out["combine_blocks"] = len(comb)
        out["combine_start"] = st(r[0] - t0 for r in comb)
        out["combine_duration"] = st(r[3] - r[0] for r in comb)
        out["combine_end"] = st(r[3] - t0 for r in comb)


def _phases(torch, run):
    """Per-block phase times (µs) of the attention kernels over one call of run(): the instrumented build's
    split stamps (block start, token loop start, loop end, block end) and combine stamps (start, end) on the
    100 MHz real-time clock; min / median / max over blocks, times relative to the first split block's start.
    With GEMV stamps in the build, the same for the last launch of each GEMV kind (block start, input prologue,
    column sums, output store, block end)."""
    import ctypes

    from leankv_amd import _lib
    lib = _lib.load()
    if not hasattr(lib, "lkv_debug_stamps"):
        raise SystemExit("--phases needs LKV_LIBRARY=leankv_amd/libleankv_amd_stamps.so "
                         "(python -m leankv_amd.build --stamps)")
    fn = lib.lkv_debug_stamps
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
    gfn = getattr(lib, "lkv_debug_gemv_stamps", None)
    if gfn is not None:
        gfn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
    n = 8 * 16384  # [block][8 stamps]
    torch.cuda.synchronize()
    for w in (0, 1):
        assert fn(w, None, 0, 1) == 0, _lib.last_error()
    if gfn is not None:
        assert gfn(0, None, 0, 1) == 0, _lib.last_error()
    run()
    torch.cuda.synchronize()
    buf = (ctypes.c_uint64 * n)()
    out = {}
    rows = {}
    for w in (0, 1):
        assert fn(w, ctypes.cast(buf, ctypes.c_void_p), n, 0) == 0, _lib.last_error()
        rows[w] = [tuple(buf[8 * i: 8 * i + 8]) for i in range(n // 8) if buf[8 * i] and buf[8 * i + 3]]
    split = rows[0]

    def st(vals):
        vals = sorted(v * 0.01 for v in vals)  # 100 MHz ticks -> µs
        return {"min": round(vals[0], 2), "median": round(statistics.median(vals), 2), "max": round(vals[-1], 2)}
    if split:
        _split_phases(out, split, rows[1], st)
    if gfn is not None:
        names = {0: "gemv_raw_input", 1: "gemv_rmsnorm", 2: "gemv_swiglu", 3: "gemv_rmsnorm_dual",
                 5: "gemv_dense_rmsnorm"}
        for kind, name in names.items():
            assert gfn(kind, ctypes.cast(buf, ctypes.c_void_p), n, 0) == 0, _lib.last_error()
            g = [tuple(buf[8 * i: 8 * i + 8]) for i in range(n // 8) if buf[8 * i] and buf[8 * i + 3]]
            if not g:
                continue
            g0 = min(r[0] for r in g)
            by_xcc, by_slab, by_chunk = {}, {}, {}
            for r in g:
                by_xcc.setdefault(int(r[4]) & 0xF, []).append((r[3] - g0) * 0.01)
                by_slab.setdefault(int(r[6]), []).append((r[3] - g0) * 0.01)
                by_chunk.setdefault(int(r[7]), []).append((r[3] - g0) * 0.01)
            slab_med = sorted(statistics.median(v) for v in by_slab.values())
            chunk_med = sorted(statistics.median(v) for v in by_chunk.values())
            out[name] = {"blocks": len(g), "start": st(r[0] - g0 for r in g), "input_prologue": st(r[1] - r[0] for r in g),
                         "column_sums": st(r[2] - r[1] for r in g), "output": st(r[3] - r[2] for r in g),
                         "end": st(r[3] - g0 for r in g),
                         "end_median_by_xcc": {x: round(statistics.median(v), 2) for x, v in sorted(by_xcc.items())},
                         "end_median_over_slabs_min_max": [round(slab_med[0], 2), round(slab_med[-1], 2)],
                         "end_median_over_chunks_min_max": [round(chunk_med[0], 2), round(chunk_med[-1], 2)]}
    out["what"] = ("µs per block on the 100 MHz clock over one call (the last launch of each kernel), relative to "
                   "the first split block's start (GEMV kinds: to that launch's first block start); instrumented "
                   "build (LKV_STAMPS)")
    return out


def bench_tq_paged(args, torch):
    """Config 4 through pages: decode attention on a paged 3-bit cache, B=16, 32/8 heads, 4096 cold tokens
    per sequence in 16-token pages scattered over the pool by a seeded permutation, 64-token fp16 hot
    rings; one lkv_tq_paged_decode_attn call per step over 8 rotating pools.  Beside it the dense
    lkv_tq_decode_attn on the same codes laid out per sequence."""
    from leankv_amd import kernels
    from leankv_amd.turboquant.codebook import get_codebook_tensors
    from leankv_amd.turboquant.rotation import generate_rotation_matrix

    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, cold, hot, ps = 16, 32, 8, 128, 4096, 64, 16
    L = cold + hot
    npg = cold // ps
    max_pages = B * npg + 8
    cent, _ = get_codebook_tensors(D, 3, dev, torch.float32)
    PiK = generate_rotation_matrix(D, dev, torch.float32, 42)
    PiV = generate_rotation_matrix(D, dev, torch.float32, 43)
    lens = torch.full((B,), L, dtype=torch.int32, device=dev)
    seq = torch.tensor([L], dtype=torch.int32, device=dev)
    indptr = torch.arange(0, B * npg + 1, npg, dtype=torch.int32, device=dev)
    sets = []
    for s in range(8):
        g = torch.Generator(device=dev).manual_seed(700 + s)
        perm = torch.randperm(max_pages, generator=g, device=dev)[: B * npg].to(torch.int32).contiguous()
        kc = torch.randint(0, 256, (max_pages, Hkv, ps, 64), generator=g, device=dev, dtype=torch.uint8) & 0x77
        vc = torch.randint(0, 256, (max_pages, Hkv, ps, 64), generator=g, device=dev, dtype=torch.uint8) & 0x77
        kn = torch.rand(max_pages, Hkv, ps, generator=g, device=dev) * 4 + 8
        vn = torch.rand(max_pages, Hkv, ps, generator=g, device=dev) * 4 + 8
        kh = torch.randn(B, Hkv, hot, D, generator=g, device=dev).half()
        vh = torch.randn(B, Hkv, hot, D, generator=g, device=dev).half()
        q = torch.randn(B, Hq, D, generator=g, device=dev).half()
        sets.append((q, kc, kn, vc, vn, kh, vh, perm, torch.empty_like(q)))

    def launch(i):
        q, kc, kn, vc, vn, kh, vh, perm, out = sets[i]
        kernels.tq_paged_decode_attn(q, kc, kn, vc, vn, kh, vh, PiK, PiV, cent, 3, indptr, perm, lens, L, D ** -0.5,
                                     out)
    wall, _, _ = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    kmean, kmed = _kernel_time(launch, len(sets), args.steps, args.warmup, torch)
    # the same codes per sequence for the dense kernel (set 0), and the two outputs compared
    q, kc, kn, vc, vn, kh, vh, perm, out = sets[0]
    pg = perm.long().view(B, npg)
    dk = kc[pg].permute(0, 2, 1, 3, 4).reshape(B, Hkv, cold, 64).contiguous()
    dv = vc[pg].permute(0, 2, 1, 3, 4).reshape(B, Hkv, cold, 64).contiguous()
    dkn = kn[pg].permute(0, 2, 1, 3).reshape(B, Hkv, cold).contiguous()
    dvn = vn[pg].permute(0, 2, 1, 3).reshape(B, Hkv, cold).contiguous()
    dout = torch.empty_like(q)
    ws = torch.empty(kernels.decode_attn_workspace_bytes(B, Hq, Hkv, L), dtype=torch.uint8, device=dev)

    def dense(_):
        kernels.tq_decode_attn_out(q, dk, dkn, dv, dvn, kh, vh, PiK, PiV, cent, 3, seq, L, D ** -0.5, dout, ws)
    dmean, _ = _kernel_time(dense, 1, args.steps, args.warmup, torch)
    launch(0)
    torch.cuda.synchronize()
    rel = float((out.float() - dout.float()).norm() / dout.float().norm())
    alg = B * Hkv * (cold * (64 + 64 + 4 + 4) + hot * D * 2 * 2) + 2 * B * Hq * D * 2 + B * npg * 4
    achieved = alg / (kmean * 1e-3) / 1e9
    return {
        "metric": "paged packed-KV decode attention HBM GB/s (B=16, 32/8 heads, 4096 cold in 16-token pages + 64 hot)",
        "value": round(achieved, 1), "unit": "GB/s", "ms_per_step": round(wall, 5), "higher_is_better": True,
        "dtype": "3-bit codes, fp16 MFMA scores/values, fp32 softmax",
        "config": {"workload": "paged_packed_attention", "batch": B, "heads": "32/8", "cold": cold, "hot": hot,
                   "page_size": ps, "alg_bytes_per_call": alg, "sets": len(sets),
                   "dense_layout": {"kernel": "lkv_tq_decode_attn on the same codes", "us": round(dmean * 1e3, 2),
                                    "paged_over_dense": round(kmean / dmean, 3), "rel_diff": rel}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "tq_attn_split_kernel<true,false,true> + tq_attn_combine_kernel (one call)",
                     "kernel_us_mean": round(kmean * 1e3, 3), "kernel_us_median": round(kmed * 1e3, 3)},
    }


# ------------------------------------------------------------------ B > 1
def bench_batched(args, torch):
    """B=8 decode rows through one TEAL-sparse projection at the config-1 shape (W[4096,14336], each row
    x ~Laplace(0,.05) with its own mask, threshold = the 40 % quantile of row 0): one
    lkv_sparse_gemm_batched call reads the weight rows some row keeps once.  Timed beside it: 8
    single-row sparse GEMV calls (what a per-row loop over the reference's kernel does) and torch's
    dense fp16 GEMM of the same shape."""
    from leankv_amd import kernels

    dev = torch.device("cuda:0")
    B, N, Z = 8, 4096, 14336
    sets = []
    for s_ in range(args.sets):
        g = torch.Generator(device=dev).manual_seed(600 + s_)
        W = (torch.randn(N, Z, generator=g, device=dev) * 0.02).half()
        Wc = W.t().contiguous().t()
        del W
        torch.manual_seed(600 + s_)
        X = torch.distributions.Laplace(0.0, 0.05).sample((B, Z)).half().to(dev)
        t = torch.kthvalue(X[0].float().abs().cpu(), int(0.4 * Z)).values.item()
        union = int(((X.float().abs() > t).any(dim=0)).sum())
        sets.append((X, Wc, t, union, torch.empty(B, N, dtype=torch.float16, device=dev)))

    def launch(i):
        X, Wc, t, _, Y = sets[i]
        kernels.sparse_gemm_batched_out(X, Wc, t, Y)

    def per_row(i):
        X, Wc, t, _, Y = sets[i]
        for b in range(B):
            kernels.sparse_gemv_out(X[b], Wc, t, Y[b])

    def dense(i):
        X, Wc, _, _, _ = sets[i]
        return X @ Wc.t()

    wall, _, _ = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    kmean, kmed = _kernel_time(launch, len(sets), args.steps, args.warmup, torch)
    rmean, _ = _kernel_time(per_row, len(sets), max(10, args.steps // 4), args.warmup, torch)
    dmean, _ = _kernel_time(dense, len(sets), args.steps, args.warmup, torch)
    union = statistics.mean(s[3] for s in sets)
    alg = union * N * 2 + B * (Z + N) * 2
    achieved = alg / (kmean * 1e-3) / 1e9
    return {
        "metric": "batched TEAL sparse GEMM HBM GB/s (B=8, W[4096,14336], 40% sparse rows)",
        "value": round(achieved, 1), "unit": "GB/s", "ms_per_step": round(wall, 5), "higher_is_better": True,
        "dtype": "f16 (fp32 accumulate)",
        "config": {"workload": "batched_sparse_gemm", "B": B, "N": N, "Z": Z, "sparsity": 0.4,
                   "union_rows_kept": round(union, 1), "alg_bytes_per_call": round(alg), "sets": len(sets)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "sparse_gemm_batched_kernel<8, BZ> + batched_reduce_kernel (one call)",
                     "kernel_us_mean": round(kmean * 1e3, 3), "kernel_us_median": round(kmed * 1e3, 3)},
        "per_row_sparse_gemv_us": round(rmean * 1e3, 3), "speedup_vs_per_row": round(rmean / kmean, 3),
        "dense_fp16_gemm_us": round(dmean * 1e3, 3),
    }


# ------------------------------------------------------------------ paged
def bench_paged(args, torch):
    """Batch decode attention on the paged fp16 pool (the dense baseline's attention; FlashInfer's batch decode in
    the reference, paged_cache.py:194-257):
    B=16 sequences of 4096 tokens, 32 query / 8 kv heads, 16-token pages scattered over the pool (seeded
    permutation).  Beside it on the same GPU: torch SDPA over the same K/V already dense (no gather), i.e.
    what a dense fp16 cache pays for the same attention."""
    from leankv_amd import kernels

    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, L, ps = 16, 32, 8, 128, 4096, 16
    npg = L // ps
    sets = []
    for s_ in range(3):
        g = torch.Generator(device=dev).manual_seed(700 + s_)
        pool = torch.randn(B * npg, 2, ps, Hkv, D, generator=g, device=dev).half()
        perm = torch.randperm(B * npg, generator=g, device=dev).to(torch.int32)
        indptr = torch.arange(0, B * npg + 1, npg, dtype=torch.int32, device=dev)
        last = torch.full((B,), ps, dtype=torch.int32, device=dev)
        q = torch.randn(B, Hq, D, generator=g, device=dev).half()
        pg = perm.long().view(B, npg)
        K = pool[pg, 0].reshape(B, L, Hkv, D).permute(0, 2, 1, 3).contiguous()
        V = pool[pg, 1].reshape(B, L, Hkv, D).permute(0, 2, 1, 3).contiguous()
        sets.append((q, pool, indptr, perm, last, torch.empty_like(q), K, V))

    def launch(i):
        q, pool, indptr, perm, last, out, _, _ = sets[i]
        kernels.paged_decode_attn(q, pool, indptr, perm, last, L, D ** -0.5, out)

    def dense(i):
        q, _, _, _, _, _, K, V = sets[i]
        return torch.nn.functional.scaled_dot_product_attention(q.unsqueeze(2), K, V, enable_gqa=True)

    q0, _, _, _, _, out0, K0, V0 = sets[0]
    launch(0)
    ref0 = dense(0).squeeze(2).float()
    agree = float((out0.float() - ref0).norm() / ref0.norm())
    wall, _, _ = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    kmean, kmed = _kernel_time(launch, len(sets), args.steps, args.warmup, torch)
    dmean, _ = _kernel_time(dense, len(sets), args.steps, args.warmup, torch)
    alg = B * Hkv * L * D * 2 * 2 + 2 * B * Hq * D * 2
    achieved = alg / (kmean * 1e-3) / 1e9
    return {
        "metric": "paged fp16 KV decode attention HBM GB/s (B=16, 32/8 heads, 4096 tokens, 16-token pages)",
        "value": round(achieved, 1), "unit": "GB/s", "ms_per_step": round(wall, 5), "higher_is_better": True,
        "dtype": "fp16 KV, fp16 MFMA scores, fp32 softmax and value sums",
        "config": {"workload": "paged_decode_attention", "batch": B, "heads": "32/8", "tokens": L, "page_size": ps,
                   "alg_bytes_per_call": alg, "sets": len(sets)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "paged_split_kernel + paged_combine_kernel (one call)",
                     "kernel_us_mean": round(kmean * 1e3, 3), "kernel_us_median": round(kmed * 1e3, 3)},
        "dense_sdpa_us": round(dmean * 1e3, 3), "rel_diff_vs_dense_sdpa": round(agree, 6),
    }


# ------------------------------------------------------------------ prefill
def bench_prefill(args, torch):
    """Causal prefill attention of one config-5 layer over its packed 3-bit cache: B=1, 32 query / 8 kv
    heads, a 4096-token prompt (4032 cold tokens as codes + the 64-token fp16 hot window), scale
    1/sqrt(128).  Timed beside it on the same GPU: the reference's algorithm for the same call,
    dequantize the cold store to fp16, concatenate the hot window, torch's causal SDPA (cache.py:169-189,
    sdpa_attention.py:79-105).  The CPU baseline is the fp64 oracle on the same layer."""
    from leankv_amd import kernels
    from leankv_amd.turboquant.codebook import get_codebook_tensors
    from leankv_amd.turboquant.rotation import generate_rotation_matrix

    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, S, hot = 1, 32, 8, 128, 4096, 64
    cold = S - hot
    cent, _ = get_codebook_tensors(D, 3, dev, torch.float32)
    PiK = generate_rotation_matrix(D, dev, torch.float32, 42)
    PiV = generate_rotation_matrix(D, dev, torch.float32, 43)
    order = torch.tensor([p % hot for p in range(cold, S)], device=dev)
    sets = []
    for s_ in range(3):
        g = torch.Generator(device=dev).manual_seed(500 + s_)
        # 3-bit codes, two per byte (64 bytes per token), every code valid
        kc = torch.randint(0, 256, (B, Hkv, cold, 64), generator=g, device=dev, dtype=torch.uint8) & 0x77
        vc = torch.randint(0, 256, (B, Hkv, cold, 64), generator=g, device=dev, dtype=torch.uint8) & 0x77
        kn = torch.rand(B, Hkv, cold, generator=g, device=dev) * 4 + 8
        vn = torch.rand(B, Hkv, cold, generator=g, device=dev) * 4 + 8
        kh = torch.randn(B, Hkv, hot, D, generator=g, device=dev).half()
        vh = torch.randn(B, Hkv, hot, D, generator=g, device=dev).half()
        q = torch.randn(B, Hq, S, D, generator=g, device=dev).half()
        sets.append((q, kc, kn, vc, vn, kh, vh, torch.empty_like(q)))
    ws = torch.empty(kernels._lib_handle().lkv_tq_prefill_attn_workspace_bytes(B, Hq, Hkv, S, hot), dtype=torch.uint8,
                     device=dev)
    scale = D ** -0.5

    def launch(i):
        q, kc, kn, vc, vn, kh, vh, out = sets[i]
        kernels.tq_prefill_attn_out(q, kc, kn, vc, vn, kh, vh, PiK, PiV, cent, 3, S, scale, out, ws)

    def reference(i):
        q, kc, kn, vc, vn, kh, vh, _ = sets[i]
        ck = kernels.tq_dequantize(kc, kn, PiK, cent, 3, out_dtype=torch.float16)
        cv = kernels.tq_dequantize(vc, vn, PiV, cent, 3, out_dtype=torch.float16)
        K = torch.cat([ck, kh.index_select(2, order)], dim=2)
        V = torch.cat([cv, vh.index_select(2, order)], dim=2)
        return torch.nn.functional.scaled_dot_product_attention(q, K, V, is_causal=True, scale=scale, enable_gqa=True)

    # agreement with the reference path on the first set (same inputs)
    launch(0)
    ref0 = reference(0).float()
    agree = float((sets[0][7].float() - ref0).norm() / ref0.norm())
    wall, _, _ = _timed_loop(launch, len(sets), args.steps, args.warmup, torch)
    kmean, kmed = _kernel_time(launch, len(sets), args.steps, args.warmup, torch)
    rmean, _ = _kernel_time(reference, len(sets), args.steps, args.warmup, torch)
    pairs = S * (S + 1) // 2  # (query, key) pairs under the causal mask, per query head
    flops = 4 * Hq * D * pairs
    tflops = flops / (kmean * 1e-3) / 1e12
    res = {
        "metric": "packed-KV causal prefill attention TFLOP/s (one layer: 4096-token prompt, 32/8 heads)",
        "value": round(tflops, 1), "unit": "TFLOP/s", "ms_per_step": round(wall, 5), "higher_is_better": True,
        "dtype": "3-bit codes, fp16 MFMA scores/values, fp32 softmax",
        "config": {"workload": "prefill_packed_attention", "batch": B, "heads": "32/8", "prompt": S, "cold": cold,
                   "hot": hot, "flop_per_call": flops, "sets": len(sets)},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "q / hot rotations + tq_prefill_attn_kernel + output un-rotation (one call)",
                     "kernel_us_mean": round(kmean * 1e3, 3), "kernel_us_median": round(kmed * 1e3, 3)},
        "prompt_tokens_per_s_per_layer": round(S / (kmean * 1e-3), 1),
        "reference_path_gpu": {"what": "tq_dequantize (fp16) + cat(hot) + torch causal SDPA, same GPU",
                               "us_mean": round(rmean * 1e3, 3), "speedup": round(rmean / kmean, 3),
                               "rel_diff_vs_packed": round(agree, 6)},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = _cpu_prefill(torch, S, hot, D)
    return res


def _cpu_prefill(torch, S, hot, D):
    """fp64 oracle on the whole layer: per kv head, dequantize its cold store and run the causal attention
    of its 4 query heads (one kv head at a time bounds the score matrix to 0.5 GB)."""
    from oracle import turboquant as oq

    cores, model = _cpu_info()
    torch.set_num_threads(cores)
    cold = S - hot
    c, _ = oq.codebook_tensors(3)
    PiK, PiV = oq.rotation_matrix(D, 42), oq.rotation_matrix(D, 43)
    g = torch.Generator().manual_seed(7)
    dt = 0.0
    for _ in range(8):  # kv heads of one layer
        kc = (torch.randint(0, 256, (1, 1, cold, 64), generator=g, dtype=torch.uint8) & 0x77).numpy()
        vc = (torch.randint(0, 256, (1, 1, cold, 64), generator=g, dtype=torch.uint8) & 0x77).numpy()
        kn = torch.rand(1, 1, cold, generator=g) * 4 + 8
        vn = torch.rand(1, 1, cold, generator=g) * 4 + 8
        kh = torch.randn(1, 1, hot, D, generator=g).half()
        vh = torch.randn(1, 1, hot, D, generator=g).half()
        q = torch.randn(1, 4, S, D, generator=g).half()
        t = time.perf_counter()
        K = torch.cat([oq.dequantize(kc, kn, PiK, c, 3).half(), kh], dim=2)
        V = torch.cat([oq.dequantize(vc, vn, PiV, c, 3).half(), vh], dim=2)
        oq.prefill_attention(q, K, V)
        dt += time.perf_counter() - t
    return {"value": round(S / dt, 2), "unit": "prompt tokens/s per layer", "cores": cores, "kind": "port",
            "sample": "oracle fp64 (dequantize + causal attention), the whole layer (8 kv heads, 32 query "
                      "heads, 4096-token prompt); %s" % model}


def _fill_gemv_defaults(args):
    if args.steps is None:
        args.steps = 200
    if args.warmup is None:
        args.warmup = 20


# ------------------------------------------------------------------ config 5
def _kv_bytes_per_token(L, Hkv, ctx, hot, bits_row=64):
    """Packed KV read by one decode step over all layers at context ctx: per kv head and cold token 2 x (code
    row + fp32 norm), per hot token 2 x 256 B of fp16."""
    cold = max(0, ctx - hot)
    return L * Hkv * (cold * 2 * (bits_row + 4) + min(ctx, hot) * 2 * 256)


def _count_survivors(model, th, cache, tokens, torch):
    """Feed `tokens` through the HF-patched model (TEAL masks and TurboQuant cache as the engine's: the two
    paths give identical activations) and count, per projection, the inputs above its threshold.  Returns
    {proj: (kept, total)} summed over layers and tokens."""
    from leankv_amd.kernels import rms_norm

    counts = {}
    hooks, saved = [], []

    def count(name, li, thresholds):
        def hook(mod, args):
            x = args[0].detach().reshape(-1).float().abs()
            for proj in thresholds:
                t = th[li][proj]
                k, n = counts.get(proj, (0, 0))
                counts[proj] = (k + int((x > t).sum()), n + x.numel())
        return hook

    for m in model.modules():  # the engine's RMSNorm arithmetic, so masks match bit for bit
        if type(m).__name__.endswith("RMSNorm"):
            saved.append((m, m.forward))
            m.forward = (lambda x, m=m: rms_norm(x, m.weight, m.variance_epsilon))
    for li, layer in enumerate(model.model.layers):
        hooks.append(layer.self_attn.q_proj.register_forward_pre_hook(count("qkv", li, ("q_proj", "k_proj", "v_proj"))))
        hooks.append(layer.self_attn.o_proj.register_forward_pre_hook(count("o", li, ("o_proj",))))
        hooks.append(layer.mlp.register_forward_pre_hook(count("gu", li, ("gate_proj", "up_proj"))))
        hooks.append(layer.mlp.down_proj.register_forward_pre_hook(count("d", li, ("down_proj",))))
    try:
        with torch.no_grad():
            for t in tokens:
                model(torch.tensor([[t]], device=model.device), past_key_values=cache, use_cache=True)
    finally:
        for h in hooks:
            h.remove()
        for m, f in saved:
            m.forward = f
    return counts


def bench_decode(args, torch):
    from leankv_amd.engine import DenseEngine, LeanKVEngine, OwnDenseEngine, random_mistral
    from leankv_amd.teal.calibrate import calibrate_thresholds, uniform_random_sparsity
    from leankv_amd.teal.patching import apply_teal
    from leankv_amd.turboquant.attention import use_on
    from leankv_amd.turboquant.cache import TurboQuantCache
    from transformers import DynamicCache

    if args.steps is None:
        args.steps = 120
    if args.warmup is None:
        args.warmup = 8
    args.warmup = max(args.warmup, 1)  # the first step runs eagerly, then the step is captured
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    model = random_mistral(device=dev, seed=0, num_hidden_layers=args.layers)
    cfg = model.config
    _log("model built in %.1fs" % (time.perf_counter() - t0))
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, cfg.vocab_size, (1, args.prompt), generator=g).to(dev)
    # TEAL calibration at the decode's context: a prompt as long as the timed one, quantiles over its last
    # 256 positions (where the timed steps' statistics are), so the sparsity decoded is the configured one
    calib = [torch.randint(0, cfg.vocab_size, (1, args.prompt), generator=g)]
    new_tokens = args.warmup + args.steps
    max_len = args.prompt + new_tokens + 2
    L, Hkv, hid, ffn, voc = (cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.hidden_size,
                             cfg.intermediate_size, cfg.vocab_size)
    nq, nkv = cfg.num_attention_heads * 128, Hkv * 128

    def timed_decode(eng):
        """warmup steps (the first eager, then the captured graph), then `steps` timed replays; returns
        (seconds, every output token in order: each step writes its token to the engine's device history)."""
        with torch.no_grad():
            p0 = eng._host_pos
            eng.step()
            eng.capture()
            for _ in range(args.warmup - 1):
                eng.step()
            torch.cuda.synchronize()
            t = time.perf_counter()
            for _ in range(args.steps):
                eng.step()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t
        return dt, [int(x) for x in eng.hist[p0:p0 + args.warmup + args.steps].tolist()]

    def hf_generate(cache_factory, runs=2):
        """scripts/benchmark.py:68-99: generate new_tokens from the prompt on a fresh cache, prefill included;
        tok/s = generated tokens / wall time, mean over runs after a 10-token warm-up."""
        model.generation_config.eos_token_id = None
        mask = torch.ones_like(prompt)
        with torch.no_grad():
            model.generate(prompt, attention_mask=mask, max_new_tokens=10, past_key_values=cache_factory(),
                           do_sample=False, pad_token_id=0)
            rates = []
            for _ in range(runs):
                c = cache_factory()
                torch.cuda.synchronize()
                t = time.perf_counter()
                out = model.generate(prompt, attention_mask=mask, max_new_tokens=new_tokens, past_key_values=c,
                                     do_sample=False, pad_token_id=0)
                torch.cuda.synchronize()
                rates.append((out.shape[1] - prompt.shape[1]) / (time.perf_counter() - t))
                del c, out
        return round(statistics.mean(rates), 2)

    # ---- dense fp16 baselines from one prefilled fp16 cache: torch's path and this library's kernels
    # (every threshold 0, fp16 paged KV); weights are still row-major here, the own engine copies them
    dense = {}
    if not args.skip_dense:
        with torch.no_grad():
            dc = DynamicCache(config=cfg)
            out = model(prompt, past_key_values=dc, use_cache=True)
            first_dense = torch.argmax(out.logits[0, -1])
            del out
        for name, cls in (("torch", DenseEngine), ("own", OwnDenseEngine)):
            eng = cls(model, max_len)
            eng.start(first_dense, eng.load_cache(dc))
            dt_d, toks_d = timed_decode(eng)
            dense[name] = (args.steps / dt_d, toks_d)
            _log("dense fp16 (%s): %.1f tok/s" % (name, dense[name][0]))
            del eng
            torch.cuda.empty_cache()
        del dc
        dense["generate"] = hf_generate(lambda: DynamicCache(config=cfg))
        _log("HF generate, dense fp16: %.1f tok/s (prefill included)" % dense["generate"])
        torch.cuda.empty_cache()

    # ---- LeanKV: TEAL thresholds from a calibration pass, HIP kernels, TurboQuant KV
    t0 = time.perf_counter()
    with torch.no_grad():
        th = calibrate_thresholds(model, calib, uniform_random_sparsity(0.3, 0.5, seed=0),
                                  positions=slice(-min(256, args.prompt), None))
    apply_teal(model, thresholds=th, use_triton=True)

    def tq_cache():
        return TurboQuantCache(bits=args.bits, head_dim=128, num_layers=L, device=dev, max_seq_len=max_len,
                               fused_attention=True)

    cache, cache_count = tq_cache(), tq_cache()
    use_on(model, cache)
    with torch.no_grad():
        out = model(prompt, past_key_values=cache, use_cache=True)
        first = torch.argmax(out.logits[0, -1])
        model(prompt, past_key_values=cache_count, use_cache=True)
        del out
    _log("calibrate + patch + TurboQuant prefill in %.1fs" % (time.perf_counter() - t0))
    eng = LeanKVEngine(model, cache, max_len)
    eng.start(first, args.prompt)
    dt, toks = timed_decode(eng)
    tps = args.steps / dt
    ms = dt * 1e3 / args.steps
    _log("leankv: %.1f tok/s" % tps)
    # one more (untimed) step with the phase stamps: the last layer's attention launches
    phases = _phases(torch, eng.step) if args.phases else None
    del eng, cache
    torch.cuda.empty_cache()

    # ---- what the timed steps read: their tokens through the HF-patched path (the same activations, masks
    # and cache as the engine's) on a cache prefilled the same way; the warm-up positions first, uncounted
    fed = [int(first)] + toks[:-1]
    _count_survivors(model, th, cache_count, fed[:args.warmup], torch)
    counts = _count_survivors(model, th, cache_count, fed[args.warmup:], torch)
    del cache_count
    torch.cuda.empty_cache()
    row_bytes = {"q_proj": nq * 2, "k_proj": nkv * 2, "v_proj": nkv * 2, "o_proj": hid * 2, "gate_proj": ffn * 2,
                 "up_proj": ffn * 2, "down_proj": hid * 2}
    in_dim = {"q_proj": hid, "k_proj": hid, "v_proj": hid, "o_proj": nq, "gate_proj": hid, "up_proj": hid,
              "down_proj": ffn}
    w_sparse = sum(counts[p][0] * row_bytes[p] for p in row_bytes) / args.steps
    w_dense = L * sum(in_dim[p] * row_bytes[p] for p in row_bytes)
    ctx = args.prompt + args.warmup + (args.steps - 1) / 2  # mean context of the timed steps
    head = hid * voc * 2
    lkv_bytes = w_sparse + head + _kv_bytes_per_token(L, Hkv, ctx, 64, bits_row=16 * {1: 1, 2: 2}.get(args.bits, 4))
    dense_bytes = w_dense + head + L * Hkv * (ctx + 1) * 2 * 256
    sparsity = {p: round(1 - counts[p][0] / counts[p][1], 4) for p in row_bytes}

    gen_lkv_hf = hf_generate(tq_cache)
    _log("HF generate, LeanKV on the patched HF forward: %.1f tok/s (prefill included)" % gen_lkv_hf)
    from leankv_amd.engine import disable_generate_fast_path, enable_generate_fast_path

    fp = enable_generate_fast_path(model)  # what optimize_model installs for TEAL + TurboQuant
    gen_lkv = hf_generate(tq_cache)
    gen_steps = dict(fp.steps)
    disable_generate_fast_path(model)
    torch.cuda.empty_cache()
    _log("HF generate, LeanKV with the fused decode step: %.1f tok/s (prefill included), calls %s"
         % (gen_lkv, gen_steps))
    res = {
        "metric": "B=1 decode tok/s (Mistral-7B shape, 40%% sparse, %d-bit KV)" % args.bits,
        "value": round(tps, 2),
        "unit": "tok/s",
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "dtype": "f16 (fp32 accumulate)",
        "data": "synthetic: random-init weights N(0,0.02), random 4096-token prompt (seeded)",
        "config": {"workload": "config5_mistral7b_decode", "layers": L, "hidden": hid, "ffn": ffn, "heads": "32/8",
                   "vocab": voc, "prompt": args.prompt, "new_tokens": new_tokens, "batch": 1,
                   "teal_sparsity": "U[0.3,0.5] per projection, mean 0.4", "kv_bits": args.bits, "hot_window": 64},
        "step_roofline": {
            "what": "algorithmic HBM bytes of one timed decode step (weight rows above threshold, counted on the "
                    "timed tokens + packed KV + lm_head) / ms_per_step",
            "bytes_per_token": int(lkv_bytes), "achieved_GBs": round(lkv_bytes / ms / 1e6, 1),
            "frac": round(lkv_bytes / ms / 1e6 / HBM_PEAK_GBS, 4),
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / lkv_bytes, 1),
            "achieved_sparsity": sparsity,
            "mean_sparsity": round(1 - w_sparse / w_dense, 4),
        },
    }
    if dense:
        own_tps, torch_tps = dense["own"][0], dense["torch"][0]
        best = max(own_tps, torch_tps)
        res["dense_fp16"] = {
            "own_kernels": {"value": round(own_tps, 2), "unit": "tok/s",
                            "what": "the same fused step, every threshold 0, fp16 KV in 16-token pages, graph-captured",
                            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / dense_bytes, 1),
                            "frac": round(own_tps * dense_bytes / 1e9 / HBM_PEAK_GBS, 4)},
            "torch": {"value": round(torch_tps, 2), "unit": "tok/s",
                      "what": "torch F.linear + SDPA, fp16 KV, graph-captured"},
        }
        res["speedup_vs_dense"] = round(tps / best, 3)
        res["speedup_vs_dense_against"] = "own_kernels" if own_tps >= torch_tps else "torch"
        res["hf_generate"] = {
            "what": "model.generate(prompt, max_new_tokens=%d, past_key_values=fresh cache), prefill included "
                    "(scripts/benchmark.py:68-99), mean of 2 runs; leankv: optimize_model's generate fast path "
                    "(single-token calls on the fused decode step), leankv_hf_forward: the patched HF forward "
                    "for every call" % new_tokens,
            "leankv_tok_s": gen_lkv, "leankv_hf_forward_tok_s": gen_lkv_hf, "dense_fp16_tok_s": dense["generate"],
            "speedup": round(gen_lkv / dense["generate"], 3), "fast_path_calls": gen_steps}
    else:
        res["hf_generate"] = {"leankv_tok_s": gen_lkv, "leankv_hf_forward_tok_s": gen_lkv_hf,
                              "fast_path_calls": gen_steps}
    if phases:
        res["phases_last_layer"] = phases
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_decode(torch, model, th, args.prompt, bits=args.bits)
    del model
    torch.cuda.empty_cache()
    return res


def bench_generate(args, torch):
    """Batched generate (the reference's sweep, scripts/sweep.py: batch sizes 1..32, 128 new tokens from a short
    prompt): config 5's model with TEAL + TurboQuant 3-bit through optimize_model's pieces, model.generate at
    B = 4 and 16 on a fresh cache, prefill included; tok/s = B x new tokens / wall time.  Decode calls go to
    BatchedEngine (the HF forward's calls replayed as a graph; at B > 1 the reference's projections are dense)
    or, for comparison, to the patched HF forward."""
    from leankv_amd.engine import disable_generate_fast_path, enable_generate_fast_path, random_mistral
    from leankv_amd.teal.calibrate import calibrate_thresholds, uniform_random_sparsity
    from leankv_amd.teal.patching import apply_teal
    from leankv_amd.turboquant.attention import use_on
    from leankv_amd.turboquant.cache import TurboQuantCache

    dev = torch.device("cuda:0")
    new, prompt_len = 128, 32
    model = random_mistral(device=dev, seed=0, num_hidden_layers=args.layers)
    cfg = model.config
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        th = calibrate_thresholds(model, [torch.randint(0, cfg.vocab_size, (1, 512), generator=g)],
                                  uniform_random_sparsity(0.3, 0.5, seed=0))
    apply_teal(model, thresholds=th, use_triton=True)
    model.generation_config.eos_token_id = None

    def run(B, fast):
        ids = torch.randint(0, cfg.vocab_size, (B, prompt_len), generator=g).to(dev)
        mask = torch.ones_like(ids)
        cache = TurboQuantCache(bits=3, head_dim=128, num_layers=cfg.num_hidden_layers, device=dev,
                                max_seq_len=prompt_len + new + 64, fused_attention=True)
        use_on(model, cache)
        torch.cuda.synchronize()
        t = time.perf_counter()
        with torch.no_grad():
            out = model.generate(ids, attention_mask=mask, max_new_tokens=new, past_key_values=cache,
                                 do_sample=False, pad_token_id=0)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t
        assert out.shape[1] == prompt_len + new
        return B * new / dt

    batches = sorted({int(b) for b in args.batches.split(",")})
    if not batches or batches[0] < 2:
        raise SystemExit("--batches: batch sizes of at least 2 (B = 1 is --workload decode)")
    top = batches[-1]
    res_b = {}
    fp = enable_generate_fast_path(model)
    for B in batches:
        run(B, True)  # warm-up: builds and captures the engine for this batch
        fast = statistics.mean(run(B, True) for _ in range(2))
        res_b[B] = {"fast_path_tok_s": round(fast, 1)}
        _log("B=%d generate, batched engine: %.1f tok/s" % (B, fast))
    calls = dict(fp.steps)
    disable_generate_fast_path(model)
    torch.cuda.empty_cache()
    for B in ([] if args.no_hf_forward else batches):
        slow = run(B, False)
        res_b[B]["hf_forward_tok_s"] = round(slow, 1)
        res_b[B]["speedup"] = round(res_b[B]["fast_path_tok_s"] / slow, 3)
        _log("B=%d generate, patched HF forward: %.1f tok/s" % (B, slow))
    return {
        "metric": "batched generate tok/s (Mistral-7B shape, TEAL thresholds, 3-bit KV, B=%d)" % top,
        "value": res_b[top]["fast_path_tok_s"], "unit": "tok/s", "higher_is_better": True,
        "steps": 2, "warmup": 1,  # timed / warm-up generate runs per batch size (each 128 new tokens)
        "ms_per_step": round(top * 1e3 / res_b[top]["fast_path_tok_s"], 4),
        "dtype": "f16 (fp32 accumulate)", "scaling": "weak",
        "data": "synthetic: random-init weights N(0,0.02), random %d-token prompts (seeded)" % prompt_len,
        "config": {"workload": "batched_generate", "prompt": prompt_len, "new_tokens": new, "kv_bits": 3,
                   "what": "model.generate(B prompts, max_new_tokens, past_key_values=fresh TurboQuantCache), prefill "
                           "included (scripts/sweep.py); at B > 1 the reference's patched projections are dense"},
        "batches": {str(b): v for b, v in res_b.items()},
        "fast_path_calls": calls,
    }


def bench_dense(args, torch):
    """The dense fp16 baseline alone (OwnDenseEngine at config 5), prefill excluded."""
    from transformers import DynamicCache

    from leankv_amd.engine import OwnDenseEngine, random_mistral

    if args.steps is None:
        args.steps = 64
    if args.warmup is None:
        args.warmup = 4
    dev = torch.device("cuda:0")
    model = random_mistral(device=dev, seed=0, num_hidden_layers=args.layers)
    cfg = model.config
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, cfg.vocab_size, (1, args.prompt), generator=g).to(dev)
    max_len = args.prompt + args.warmup + args.steps + 2
    with torch.no_grad():
        dc = DynamicCache(config=cfg)
        out = model(prompt, past_key_values=dc, use_cache=True)
        first = torch.argmax(out.logits[0, -1])
        del out
    eng = OwnDenseEngine(model, max_len)
    eng.start(first, eng.load_cache(dc))
    del dc
    torch.cuda.empty_cache()
    with torch.no_grad():
        eng.step()
        eng.capture()
        for _ in range(args.warmup - 1):
            eng.step()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(args.steps):
            eng.step()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t
    L, Hkv, hid, ffn, voc = (cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.hidden_size,
                             cfg.intermediate_size, cfg.vocab_size)
    nq, nkv = cfg.num_attention_heads * 128, Hkv * 128
    ctx = args.prompt + args.warmup + (args.steps - 1) / 2
    dense_bytes = L * 2 * (hid * (nq + 2 * nkv) + nq * hid + 3 * hid * ffn) + hid * voc * 2 + L * Hkv * (ctx + 1) * 512
    ms = dt * 1e3 / args.steps
    return {
        "metric": "B=1 dense fp16 decode tok/s (Mistral-7B shape, this library's kernels, threshold 0)",
        "value": round(args.steps / dt, 2), "unit": "tok/s", "ms_per_step": round(ms, 4), "higher_is_better": True,
        "dtype": "f16 (fp32 accumulate)",
        "config": {"workload": "config5_dense_fp16_own_kernels", "layers": L, "prompt": args.prompt, "batch": 1},
        "step_roofline": {"bytes_per_token": int(dense_bytes), "achieved_GBs": round(dense_bytes / ms / 1e6, 1),
                          "frac": round(dense_bytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                          "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / dense_bytes, 1)},
    }


def _log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


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
    # stdout carries exactly one JSON line: whatever the workload prints (the TEAL patching notice,
    # progress) goes to stderr
    real_stdout = sys.stdout
    sys.stdout = sys.stderr
    try:
        res = _run_workload(args, torch)
    finally:
        sys.stdout = real_stdout
    out = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup}
    out.update(res)
    out.setdefault("scaling", "weak")
    out.setdefault("vs_baseline", None)
    out.setdefault("data", "synthetic (seeded)")
    print(json.dumps(out))


def _run_workload(args, torch):
    if args.workload == "decode":
        res = bench_decode(args, torch)
        # roofline block: the dominant kernel of the decode step (fused gate/up GEMV)
        if not args.no_roofline:
            res["roofline"] = roofline_gateup(args, torch)
    else:
        _fill_gemv_defaults(args)
        fn = {"generate": bench_generate, "dense": bench_dense, "gemv": bench_gemv, "mlp": bench_mlp, "copy": bench_copy, "quant": bench_quant,
              "attn": bench_attn, "prefill": bench_prefill, "batched": bench_batched,
              "paged": bench_paged, "tqpaged": bench_tq_paged, "prod": bench_prod}.get(args.workload)
        if fn is None:
            print("bench.py: workload %s is not implemented yet" % args.workload, file=sys.stderr)
            sys.exit(2)
        res = fn(args, torch)
    return res


if __name__ == "__main__":
    main()
