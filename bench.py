"""Benchmark of the dilution-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                    [--decode-steps K] [--no-decode] [--no-cpu-baseline]

Prints ONE JSON line.  The headline workload (default ``train16k``) is the
operator's training step, fwd+bwd through ``dilution.kernels.dilution_attention``
(the autograd drop-in), at B=1 H=16 T=16384 d=64 bf16 with q,k ~ 0.5 N(0,1),
v, dO ~ N(0,1), inputs resident in HBM before the timed region.  ``value`` is
algorithmic TFLOP/s, 7 B H T^2 d per step (the causal flash-attention
fwd+bwd count: forward 2 products, backward 5 including one recompute).

The same line carries
  * ``roofline`` for the step's dominant kernel: its algorithmic FLOPs per
    launch over its average HIP-event duration inside the timed region;
  * ``kernels``: per-kernel launches and average milliseconds;
  * ``decode``: the cached decode step at 128K context (B=16 H=16 d=64 bf16),
    HBM GB/s over B H L (4d + 8) algorithmic bytes per step, with its own
    roofline object;
  * ``cpu_baseline``: the fp32 CPU oracle (torch eager, the reference
    formula) timed on this host's cores on a bounded sample of the workload.
One GPU only: ``--gpus`` above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "dilution-attention_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "dilution-attn fwd+bwd TFLOP/s & decode HBM GB/s at T=16K, % of MI355X peak"
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3       # MI355X fp32 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E

# Training-step workloads: (batch, heads, seq, head_dim)
WORKLOADS = {
    "train16k": (1, 16, 16384, 64),
    "train2k": (8, 16, 2048, 64),
}

# Algorithmic products (each B H T^2 d FLOPs causal) that each kernel of the
# training step carries; they sum to the 7 of the step.  Recomputed products
# (extra score products, the pk product, the dk correction) count zero.
ALGO_PRODUCTS = {
    "fwd_stats": 1,     # Q K^T (row statistics)
    "fwd_out": 1,       # share @ V
    "bwd_key": 4,       # Q K^T recompute, dO V^T, A^T dO (dv), (p dp)^T Q (dk)
    "bwd_query": 1,     # (p dp) K (dq)
    "bwd_dkcorr": 0,
    "bwd_rows": 0,
    "fwd_scan": 0,
    "prep": 0,
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="train16k")
    ap.add_argument("--decode-steps", type=int, default=50)
    ap.add_argument("--decode-context", type=int, default=131072)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def synthetic_training_inputs(shape, dev, seed=2):
    """q, k ~ 0.5 N(0,1), v, dO ~ N(0,1) from a CPU generator, cast to bf16
    and copied to the GPU before any timing."""
    import torch

    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(*shape, generator=g) * 0.5).to(torch.bfloat16)
    k = (torch.randn(*shape, generator=g) * 0.5).to(torch.bfloat16)
    v = torch.randn(*shape, generator=g).to(torch.bfloat16)
    do = torch.randn(*shape, generator=g).to(torch.bfloat16)
    return [t.to(dev) for t in (q, k, v, do)]


def bench_training(args, dev):
    import torch

    from dilution import _hip, kernels

    batch, heads, seq, d = WORKLOADS[args.workload]
    q, k, v, do = synthetic_training_inputs((batch, heads, seq, d), dev)
    xs = [t.requires_grad_(True) for t in (q, k, v)]

    def step():
        for x in xs:
            x.grad = None
        out = kernels.dilution_attention(*xs, dot_precision="bf16")
        out.backward(do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"{args.workload}: warmup {args.warmup} done")

    torch.cuda.synchronize()
    with _hip.kernel_timing() as kt:
        t0 = time.perf_counter()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            step()
        stop.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_event = start.elapsed_time(stop) / args.steps
    ms = max(ms_event, wall * 1e3 / args.steps)
    log(f"{args.workload}: {args.steps} timed steps, {ms:.3f} ms/step")

    unit = batch * heads * seq * seq * d            # one causal product: B H T^2 d FLOPs
    flops = 7.0 * unit
    tflops = flops / (ms * 1e-3) / 1e12
    per_kernel = {name: {"launches": n, "avg_ms": tot / max(n, 1), "ms_per_step": tot / args.steps}
                  for name, (n, tot) in kt.result.items()}
    dom = max(per_kernel, key=lambda nm: per_kernel[nm]["ms_per_step"])
    dom_flops = ALGO_PRODUCTS.get(dom, 0) * unit     # per launch: every kernel runs once per step
    dom_ms = per_kernel[dom]["avg_ms"]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    roof = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
            "algorithmic_flops_per_launch": dom_flops, "avg_launch_ms": round(dom_ms, 4)}
    for rec in per_kernel.values():
        rec["avg_ms"] = round(rec["avg_ms"], 4)
        rec["ms_per_step"] = round(rec["ms_per_step"], 4)
    return dict(ms=ms, value=tflops, flops=flops, roofline=roof, kernels=per_kernel,
                shape=(batch, heads, seq, d))


def bench_decode(args, dev):
    """Cached decode at context L (BASELINE configs[3] shape B16 H16 d64 bf16):
    synthetic K/V caches and a non-negative demand vector resident in HBM."""
    import torch

    from dilution import _hip, kernels

    batch, heads, d, length = 16, 16, 64, args.decode_context
    g = torch.Generator(device=dev).manual_seed(4)
    kc = torch.randn(batch, heads, length, d, device=dev, generator=g, dtype=torch.bfloat16)
    vc = torch.randn(batch, heads, length, d, device=dev, generator=g, dtype=torch.bfloat16)
    com = torch.rand(batch, heads, length, device=dev, generator=g) * 4.0
    com[..., length - 1] = 0.0
    q1 = torch.randn(batch, heads, 1, d, device=dev, generator=g, dtype=torch.bfloat16)

    def step():
        kernels.dilution_decode_step(q1, kc, vc, com, length)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    with _hip.kernel_timing() as kt:
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.decode_steps):
            step()
        stop.record()
        torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.decode_steps
    nbytes = batch * heads * length * (4 * d + 8)
    gbs = nbytes / (ms * 1e-3) / 1e9
    per_kernel = {name: {"launches": n, "avg_ms": round(tot / max(n, 1), 4)}
                  for name, (n, tot) in kt.result.items()}
    kern_ms = sum(tot for (_, tot) in kt.result.values()) / args.decode_steps
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    log(f"decode L={length}: {ms:.3f} ms/step, {gbs:.0f} GB/s")
    return {"metric": "decode HBM GB/s", "value": round(gbs, 1), "unit": "GB/s",
            "ms_per_step": round(ms, 4), "steps": args.decode_steps,
            "config": {"workload": "C4 cached decode", "batch": batch, "heads": heads,
                       "context": length, "head_dim": d, "dtype": "bf16"},
            "roofline": {"kernel": "dec_stats+dec_apply+dec_finish (one step)", "bound": "hbm",
                         "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                         "algorithmic_bytes_per_step": nbytes},
            "kernels": per_kernel}


def cpu_baseline(shape):
    """The fp32 CPU oracle, fwd+bwd through torch autograd, on one (batch,
    head) slice of the workload (the slices are independent and identical in
    cost), timed on this host's cores."""
    import torch

    from oracle import dilution_oracle as orc

    threads = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        threads = min(threads, int(env))
    torch.set_num_threads(threads)
    _, _, seq, d = shape
    q, k, v, do = orc.make_inputs((1, 1, seq, d), seed=2, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    xs = [t.float().requires_grad_(True) for t in (q, k, v)]
    t0 = time.perf_counter()
    out = orc.attention_fp32(*xs)
    out.backward(do.float())
    dt = time.perf_counter() - t0
    flops = 7.0 * seq * seq * d
    log(f"cpu baseline: one slice T={seq} fwd+bwd in {dt:.2f} s on {threads} threads")
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "seconds": round(dt, 2),
            "sample": f"fp32 torch-eager oracle fwd+bwd on 1 of {shape[0] * shape[1]} (batch, head) "
                      f"slices, T={seq} d={d}"}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the dilution-attention "
              "path here runs on a single MI355X, see DESIGN.md for how it would shard",
              file=sys.stderr)
        return 2
    import torch

    from dilution import kernels

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if not kernels.HAS_HIP:
        print("libdilution_hip.so is not built (run __graft_entry__.build())", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    tr = bench_training(args, dev)
    batch, heads, seq, d = tr["shape"]
    line = {
        "metric": METRIC,
        "value": round(tr["value"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(tr["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (q,k ~ 0.5 N(0,1), v, dO ~ N(0,1), CPU RNG seed 2, bf16)",
        "config": {"workload": f"{args.workload}: operator fwd+bwd B{batch} H{heads} T{seq} d{d}",
                   "batch": batch, "heads": heads, "seq_len": seq, "head_dim": d,
                   "parallelism": "none (1 GPU)"},
        "pct_of_peak": round(100.0 * tr["value"] / PEAK_BF16_TFLOPS, 2),
        "roofline": tr["roofline"],
        "kernels": tr["kernels"],
    }
    if not args.no_decode:
        torch.cuda.empty_cache()
        line["decode"] = bench_decode(args, dev)
    if not args.no_cpu_baseline:
        torch.cuda.empty_cache()
        line["cpu_baseline"] = cpu_baseline(tr["shape"])
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
