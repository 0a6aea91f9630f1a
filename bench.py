#!/usr/bin/env python3
"""Benchmark of the sharded AdamW + global-norm clip step on one flat shard.

Workload: one FSDP rank of Llama-3-8B at W=8, i.e. a 1,003,782,656-element fp32
flat shard (8,030,261,248 / 8, no padding), p ~ N(0, 0.02), g ~ N(0, 1e-4), m = v = 0,
AdamW lr 3e-4, betas (0.9, 0.95), eps 1e-8, weight decay 0.1, global-norm clip at
1.0 (the norm is about 3.17, so clipping is active).  Inputs are generated on the
device before timing and stay resident in HBM.

One step = the drop-in call sequence ``clip_grad_norm(1.0); step()`` of
``ShardedOptimizer`` with the clip deferred into the update: the fp64 norm pass
(reads g, 4 B/element) and the fused clip + AdamW pass (reads p, g, m, v and writes
p, m, v: 28 B/element), 32 B/element in all.

Prints one JSON line on stdout; progress goes to stderr.  ``value`` is params/s of
the whole step.  ``roofline`` is for the dominant kernel (the fused AdamW): its
algorithmic bytes per launch (28 * numel) over its mean duration, taken from HIP
events recorded on the launch stream around every timed launch.  ``traffic`` is
read from the committed rocprofv3 counter summary when present.  ``cpu_baseline``
times the reference's own CPU op sequence (torch CPU ops, torch.optim.AdamW) on a
bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "build-your-own-hybrid-distributed-training_amd"))
sys.path.insert(0, HERE)

LLAMA3_8B_PARAMS = 8_030_261_248
WORLD = 8
SHARD_NUMEL = LLAMA3_8B_PARAMS // WORLD  # 1,003,782,656
LR, BETAS, EPS, WD, MAX_NORM = 3e-4, (0.9, 0.95), 1e-8, 0.1, 1.0
HBM_PEAK_GBPS = 8000.0
BYTES_NORM = 4  # read g
BYTES_ADAMW = 28  # read p, g, m, v; write p, m, v
TRAFFIC_SUMMARY = os.path.join(HERE, "profiles", "adamw_llama3_8b_w8_shard_traffic.json")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--numel", type=int, default=SHARD_NUMEL, help="shard size (default: Llama-3-8B / 8)")
    ap.add_argument("--cpu-numel", type=int, default=1 << 26, help="CPU-baseline sample size")
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument(
        "--calibrate-copy",
        action="store_true",
        help="instead of the benchmark, run the library's interval-copy kernel over a 1 GiB fp32 "
        "buffer (known traffic: 1 GiB read + 1 GiB written per launch) to scale HBM counters",
    )
    return ap.parse_args()


def calibrate_copy() -> int:
    """Three launches of hbt_copy_intervals moving one 1 GiB fp32 buffer into another."""
    import torch

    from hybrid_training_amd import _native

    device = torch.device("cuda", 0)
    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        plan = _native.CopyPlan(device)
        plan.add(src, 0, dst, 0, n)
        plan.run(src_dtype=torch.float32, dst_dtype=torch.float32)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "hbt_copy_intervals", "bytes_read": 4 * n, "bytes_written": 4 * n,
                      "launches": 3, "ok": bool(torch.equal(src, dst))}), flush=True)
    return 0


def cpu_baseline(numel: int, steps: int) -> dict:
    import torch

    from oracle.cpu_reference_path import ReferenceCpuStep

    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    ref = ReferenceCpuStep(numel, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    ref.prepare()
    ref.step(MAX_NORM)  # warm-up
    elapsed = 0.0
    for _ in range(steps):
        ref.prepare()
        t0 = time.perf_counter()
        ref.step(MAX_NORM)
        elapsed += time.perf_counter() - t0
    per_step = elapsed / steps
    return {
        "value": numel / per_step,
        "unit": "params/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"{numel} fp32 elements (of the {SHARD_NUMEL}-element shard), {steps} timed steps after "
            f"1 warm-up: fp64 norm + clip + torch.optim.AdamW(foreach=False).step on CPU, "
            f"{threads} threads; host has {os.cpu_count()} logical CPUs"
        ),
        "ms_per_step": per_step * 1e3,
    }


def read_traffic() -> float | None:
    try:
        with open(TRAFFIC_SUMMARY, encoding="utf-8") as f:
            data = json.load(f)
        return float(data["adamw_hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main() -> int:
    args = parse_args()
    if args.calibrate_copy:
        return calibrate_copy()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build runs one rank's share of the work on one "
            "device and issues no collectives; --gpus must be 1",
            file=sys.stderr,
        )
        return 2

    import torch

    from hybrid_training_amd import GroupHandle, OptimizerConfig, ShardedOptimizer

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    device = torch.device("cuda", 0)
    n = args.numel
    log(f"allocating a {n}-element fp32 shard (p, g, m, v: {16 * n / 1e9:.1f} GB)")
    gen = torch.Generator(device=device).manual_seed(0)
    param = torch.nn.Parameter(torch.randn(n, device=device, generator=gen).mul_(0.02))
    grad = torch.randn(n, device=device, generator=torch.Generator(device=device).manual_seed(1)).mul_(1e-4)
    optimizer = ShardedOptimizer(
        [param],
        OptimizerConfig(name="adamw", learning_rate=LR, betas=BETAS, eps=EPS, weight_decay=WD),
        # This rank's share of the norm: an FSDP flat shard's elements carry weight
        # G / W = 1, the same as a one-rank group's.
        norm_group=GroupHandle.trivial("world"),
        device=device,
        defer_clip=True,
    )
    # state tensors allocated up front, as after the first step
    param.grad = grad
    stream = torch.cuda.current_stream(device)

    def one_step(events=None):
        if events is not None:
            events[0].record(stream)
        norm = optimizer.clip_grad_norm(MAX_NORM)
        if events is not None:
            events[1].record(stream)
        optimizer.step()
        if events is not None:
            events[2].record(stream)
        param.grad = grad  # zero_grad(set_to_none) + a new backward, without the backward
        return norm

    log(f"warm-up: {args.warmup} steps")
    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        norm = one_step(events[k])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    norm_value = float(norm)

    norm_ms = sum(e[0].elapsed_time(e[1]) for e in events) / args.steps
    adamw_ms = sum(e[1].elapsed_time(e[2]) for e in events) / args.steps
    ms_per_step = wall * 1e3 / args.steps
    adamw_gbps = BYTES_ADAMW * n / (adamw_ms * 1e-3) / 1e9
    step_gbps = (BYTES_NORM + BYTES_ADAMW) * n / (ms_per_step * 1e-3) / 1e9
    log(f"norm {norm_value:.6f}; {ms_per_step:.3f} ms/step (norm {norm_ms:.3f} ms, adamw {adamw_ms:.3f} ms)")

    result = {
        "metric": "sharded AdamW+clip step: params/s and HBM GB/s (% of peak) on 1 flat shard",
        "value": n / (ms_per_step * 1e-3),
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (device-generated, seeds 0 and 1)",
        "config": {
            "workload": "Llama-3-8B FSDP rank shard at W=8: fused global-norm clip + AdamW",
            "shard_numel": n,
            "optimizer": {"lr": LR, "betas": list(BETAS), "eps": EPS, "weight_decay": WD},
            "max_grad_norm": MAX_NORM,
            "bytes_per_param": BYTES_NORM + BYTES_ADAMW,
        },
        "step_hbm_gbps": step_gbps,
        "step_frac_of_peak": step_gbps / HBM_PEAK_GBPS,
        "kernel_ms": {"grad_norm": norm_ms, "adamw": adamw_ms},
        "grad_norm": norm_value,
        "roofline": {
            "bound": "hbm",
            "achieved": adamw_gbps,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": adamw_gbps / HBM_PEAK_GBPS,
            "traffic": read_traffic(),
        },
        "cpu_baseline": None,
    }
    del optimizer, param, grad
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        log(f"CPU baseline on {args.cpu_numel} elements")
        result["cpu_baseline"] = cpu_baseline(args.cpu_numel, args.cpu_steps)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
