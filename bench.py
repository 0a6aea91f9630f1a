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
bounded sample of the same workload.  The other workloads (``--workload``) carry a
``cpu_baseline`` of the reference's op sequence for that workload too, on a bounded
sample stated in the line; the loss scaler's clean steps carry none, because torch's
CPU AdamW refuses bf16 gradients on fp32 parameters.
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
SECONDARY_TRAFFIC = os.path.join(HERE, "profiles", "secondary_workloads_traffic.json")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--numel", type=int, default=SHARD_NUMEL, help="shard size (default: Llama-3-8B / 8)")
    ap.add_argument("--cpu-numel", type=int, default=1 << 28, help="CPU-baseline sample size")
    ap.add_argument("--cpu-steps", type=int, default=20,
                    help="timed CPU-baseline steps (about 11 s of CPU work at the default size)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument(
        "--workload",
        choices=["adamw", "buckets", "reshard", "scaler", "fsdp", "inplace_clip", "torch_adamw", "sgd", "offload",
                 "param_offload", "checkpoint", "copy_ceiling", "lowp", "mlp"],
        default="adamw",
        help="adamw (default): the Llama-3-8B W=8 shard step above; buckets: GPT-2-small DDP bucket "
        "pack + AVG divide at W=8; reshard: Llama-3-8B bf16 flat shards W=4 -> W=8 and W=2; scaler: "
        "one Llama-3-70B W=8 rank shard with bf16 gradients, loss scale 2^16, clip and AdamW; fsdp: "
        "Llama-3-8B FSDP pack, unpack, gradient local share and no_sync accumulation at W=8; inplace_clip: the headline step with "
        "the reference's in-place clip; torch_adamw: the headline step with stock torch GPU kernels; sgd: "
        "the headline shard with SGD (momentum 0.9); offload: the headline step with AdamW state in pinned "
        "host memory; param_offload: the headline shard as an FSDP unit with the shard, its gradient and "
        "its AdamW state in pinned host memory; checkpoint: Llama-3-8B bf16 saved by 4 FSDP ranks and loaded back at W=8; "
        "copy_ceiling: torch's device-to-device copy against the interval copy on 1 and 16 GiB; lowp: the headline "
        "shard with bf16 masters (AdamW and SGD); mlp: the reference's 1,857-parameter MLP as FSDP units at W=2 and 4, "
        "the per-rank tail (local share + clip + AdamW)",
    )
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


def _time_cpu_step(numel: int, steps: int, threads: int, momentum: float | None = None, dtype=None) -> float:
    """Mean seconds of the reference's CPU step on ``numel`` elements with ``threads`` threads
    (AdamW, or SGD with ``momentum``; fp32 unless ``dtype``)."""
    import torch

    from oracle.cpu_reference_path import ReferenceCpuStep

    torch.set_num_threads(threads)
    ref = ReferenceCpuStep(numel, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, momentum=momentum,
                           dtype=dtype or torch.float32)
    ref.prepare()
    ref.step(MAX_NORM)  # warm-up
    elapsed = 0.0
    for _ in range(steps):
        ref.prepare()
        t0 = time.perf_counter()
        ref.step(MAX_NORM)
        elapsed += time.perf_counter() - t0
    del ref
    return elapsed / steps


def _cpu_step_line(numel: int, steps: int, momentum: float | None = None, dtype=None) -> dict:
    """The reference's clipped CPU step (AdamW, or SGD with ``momentum``) on a bounded sample."""
    seconds = _time_cpu_step(numel, steps, _cpu_threads(), momentum, dtype)
    name = "torch.optim.AdamW" if momentum is None else f"torch.optim.SGD(momentum={momentum})"
    kind = "fp32" if dtype is None else str(dtype).replace("torch.", "")
    return _cpu_line(numel, seconds, "params/s",
                     f"{numel} {kind} elements, {steps} timed steps after 1 warm-up: fp64 norm + in-place clip + "
                     f"{name}(foreach=False).step")


def cpu_baseline(numel: int, steps: int) -> dict:
    """The reference's CPU step timed on this host: all cores (up to 16), then one thread.

    The reference's own harness pins one thread per rank process; the all-core figure
    is the stronger baseline and is the reported ``value``.
    """
    threads = min(os.cpu_count() or 1, 16)
    per_step = _time_cpu_step(numel, steps, threads)
    single_numel = max(1, numel // 4)
    single = _time_cpu_step(single_numel, max(1, steps // 2), 1)
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
        "single_thread": {
            "value": single_numel / single,
            "unit": "params/s",
            "cores": 1,
            "sample": f"{single_numel} fp32 elements, {max(1, steps // 2)} timed steps after 1 warm-up",
            "ms_per_step": single * 1e3,
        },
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
            "bench.py measures one GPU: the library runs one rank's share of the work on one "
            "device and issues no collectives; --gpus must be 1",
            file=sys.stderr,
        )
        return 2
    if args.workload != "adamw":
        global _WITH_CPU
        _WITH_CPU = not args.no_cpu_baseline
        status = SECONDARY[args.workload](args.steps, args.warmup)
        _settle()
        return status

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
            "clip": "multiplier applied inside the fused update (defer_clip): parameters and state bitwise "
                    "those of the in-place .grad clip, which --workload inplace_clip measures",
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
    _settle()
    return 0


def _settle() -> None:
    """Wait for every queued kernel and copy (a streamed pass may leave non-blocking copies
    to pinned host memory in flight) before the process starts to exit."""
    import torch

    if torch.cuda.is_initialized():
        torch.cuda.synchronize()


# ---------------------------------------------------------------------------------------
# Secondary workloads (one JSON line each; the default run is the AdamW shard step).
# ---------------------------------------------------------------------------------------
def _time_events(fn, steps: int, warmup: int) -> float:
    """Mean milliseconds of fn() over `steps` runs, HIP events on the current stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def _gpt2_small_shapes():
    d, vocab, ctx = 768, 50257, 1024
    named = [("wte.weight", (vocab, d)), ("wpe.weight", (ctx, d))]
    for i in range(12):
        p = f"h.{i}."
        named += [(p + "ln_1.weight", (d,)), (p + "ln_1.bias", (d,)),
                  (p + "attn.c_attn.weight", (d, 3 * d)), (p + "attn.c_attn.bias", (3 * d,)),
                  (p + "attn.c_proj.weight", (d, d)), (p + "attn.c_proj.bias", (d,)),
                  (p + "ln_2.weight", (d,)), (p + "ln_2.bias", (d,)),
                  (p + "mlp.c_fc.weight", (d, 4 * d)), (p + "mlp.c_fc.bias", (4 * d,)),
                  (p + "mlp.c_proj.weight", (4 * d, d)), (p + "mlp.c_proj.bias", (d,))]
    return named + [("ln_f.weight", (d,)), ("ln_f.bias", (d,))]


def _llama3_shapes(layers, d, ffn, kv_dim, vocab):
    named = [("model.embed_tokens.weight", (vocab, d))]
    for i in range(layers):
        p = f"model.layers.{i}."
        named += [(p + "self_attn.q_proj.weight", (d, d)), (p + "self_attn.k_proj.weight", (kv_dim, d)),
                  (p + "self_attn.v_proj.weight", (kv_dim, d)), (p + "self_attn.o_proj.weight", (d, d)),
                  (p + "mlp.gate_proj.weight", (ffn, d)), (p + "mlp.up_proj.weight", (ffn, d)),
                  (p + "mlp.down_proj.weight", (d, ffn)), (p + "input_layernorm.weight", (d,)),
                  (p + "post_attention_layernorm.weight", (d,))]
    return named + [("model.norm.weight", (d,)), ("lm_head.weight", (vocab, d))]


def _secondary_traffic(workload: str, labels: list[str], launches: list[int]) -> float | None:
    """HBM bytes per step from the committed counter summary: sum of launches x bytes per launch."""
    try:
        with open(SECONDARY_TRAFFIC, encoding="utf-8") as f:
            data = json.load(f)[workload]
        return sum(k * float(data[label]["hbm_bytes_per_launch"]) for label, k in zip(labels, launches))
    except (OSError, KeyError, ValueError):
        return None


def _emit(metric, unit, value, ms, steps, warmup, dtype, workload, bytes_per_run, extra=None, traffic=None,
          cpu_baseline=None):
    """One JSON line for a secondary workload.  Its roofline is per step: algorithmic bytes
    of the step over the step time, and HBM traffic per step (``traffic_per`` says so).
    ``cpu_baseline``: the reference's op sequence for the workload timed on this host's
    cores (a bounded sample, in the same unit as ``value``), or None."""
    gbps = bytes_per_run / (ms * 1e-3) / 1e9
    line = {
        "metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (device-generated)", "config": {"workload": workload},
        "roofline": {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": gbps / HBM_PEAK_GBPS, "traffic": traffic, "traffic_per": "step"},
        "cpu_baseline": cpu_baseline,
    }
    if extra:
        line["config"].update(extra)
    print(json.dumps(line), flush=True)


#: Whether the secondary workloads time their CPU baselines (``--no-cpu-baseline`` clears it).
_WITH_CPU = True


def _cpu_threads() -> int:
    return min(os.cpu_count() or 1, 16)


def _cpu_time(fn, reps: int) -> float:
    """Mean seconds of ``fn()`` on this host's cores (up to 16), after one warm-up call."""
    import torch

    torch.set_num_threads(_cpu_threads())
    fn()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps


def _cpu_line(units_per_run: float, seconds: float, unit: str, sample: str) -> dict:
    """A ``cpu_baseline`` object: ``units_per_run`` units of the workload per ``seconds``."""
    threads = _cpu_threads()
    return {"value": units_per_run / seconds, "unit": unit, "cores": threads, "kind": "port",
            "sample": f"{sample}; torch CPU ops, {threads} threads, host has {os.cpu_count()} logical CPUs",
            "ms_per_step": seconds * 1e3}


def bench_buckets(steps: int, warmup: int) -> int:
    """GPT-2 small (124,439,808 fp32), 25 MiB buckets, pack + AVG divide at W=8: 8 B/param."""
    import torch

    from hybrid_training_amd import BucketedGradients, DDPConfig, GroupHandle

    device = torch.device("cuda", 0)
    named = [(n, torch.nn.Parameter(torch.empty(s, device=device))) for n, s in _gpt2_small_shapes()]
    gen = torch.Generator(device=device).manual_seed(2)
    grads = [torch.randn(p.shape, device=device, generator=gen).mul_(1e-3) for _, p in named]
    ddp = BucketedGradients(named, GroupHandle.local_view("data_parallel", 8, 0), DDPConfig(bucket_cap_mb=25.0))
    n = sum(p.numel() for _, p in named)

    def run():
        for (_, p), g in zip(named, grads):
            p.grad = g
        ddp.pack()

    ms = _time_events(run, max(steps, 20), max(warmup, 3))
    cpu = None
    if _WITH_CPU:
        from oracle.cpu_reference_path import pack_buckets

        host = {id(p): g.cpu() for (_, p), g in zip(named, grads)}
        buckets = [(torch.empty(b.layout.total_numel, dtype=torch.float32),
                    [(b.layout.offsets[i], host[id(q)]) for i, q in enumerate(b.parameters)]) for b in ddp.buckets]
        cpu = _cpu_line(n, _cpu_time(lambda: pack_buckets(buckets, 8), 5), "params/s",
                        f"all {n} gradients into the {len(buckets)} buckets, copy + div_(8) per bucket, "
                        "5 timed runs after 1 warm-up")
        del host, buckets
    _emit("DDP bucket pack + AVG divide: params/s", "params/s", n / (ms * 1e-3), ms, max(steps, 20),
          max(warmup, 3), "f32", "GPT-2 small gradients, 17 buckets of <= 25 MiB, W=8", 8 * n,
          {"params": n, "buckets": len(ddp.buckets), "bytes_per_param": 8},
          _secondary_traffic("buckets", ["pack + AVG divide (one launch)"], [1]), cpu)
    # The same model in bf16: bf16 gradients packed into bf16 buckets (read 2 B + write 2 B).
    del ddp
    named16 = [(name, torch.nn.Parameter(torch.empty(p.shape, dtype=torch.bfloat16, device=device)))
               for name, p in named]
    grads16 = [g.to(torch.bfloat16) for g in grads]
    ddp16 = BucketedGradients(named16, GroupHandle.local_view("data_parallel", 8, 0), DDPConfig(bucket_cap_mb=25.0))

    def run16():
        for (_, p), g in zip(named16, grads16):
            p.grad = g
        ddp16.pack()

    ms = _time_events(run16, max(steps, 20), max(warmup, 3))
    cpu = None
    if _WITH_CPU:
        from oracle.cpu_reference_path import pack_buckets

        host = {id(p): g.cpu() for (_, p), g in zip(named16, grads16)}
        buckets = [(torch.empty(b.layout.total_numel, dtype=torch.bfloat16),
                    [(b.layout.offsets[i], host[id(q)]) for i, q in enumerate(b.parameters)]) for b in ddp16.buckets]
        cpu = _cpu_line(n, _cpu_time(lambda: pack_buckets(buckets, 8), 5), "params/s",
                        f"all {n} bf16 gradients into the {len(buckets)} buckets, copy + div_(8) per bucket, "
                        "5 timed runs after 1 warm-up")
        del host, buckets
    _emit("DDP bucket pack + AVG divide, bf16 gradients: params/s", "params/s", n / (ms * 1e-3), ms, max(steps, 20),
          max(warmup, 3), "bf16", f"GPT-2 small bf16 gradients, {len(ddp16.buckets)} buckets of <= 25 MiB, W=8", 4 * n,
          {"params": n, "buckets": len(ddp16.buckets), "bytes_per_param": 4},
          _secondary_traffic("buckets", ["bf16 gradients: pack + AVG divide (one launch)"], [1]), cpu)
    return 0


def bench_reshard(steps: int, warmup: int) -> int:
    """Llama-3-8B bf16 (8,030,261,248) saved by 4 ranks, loaded by 8 and by 2: 4 B/elem per re-slice."""
    import torch

    from hybrid_training_amd import (DeviceShardCache, PieceLayout, ShardRange, ShardRecord, TensorRecord,
                                     intersect_ranges, load_flat_shard, shard_filename)

    device = torch.device("cuda", 0)
    shapes = _llama3_shapes(32, 4096, 14336, 1024, 128256)
    numels = [int(torch.Size(s).numel()) for _, s in shapes]
    total = sum(numels)
    s_src = total // 4
    gen = torch.Generator(device=device).manual_seed(4)
    shards = [torch.randint(-(2**15), 2**15, (s_src,), dtype=torch.int16, device=device, generator=gen)
              .view(torch.bfloat16) for _ in range(4)]
    records, cache, cursor = {}, DeviceShardCache(), 0
    for (name, shape), numel in zip(shapes, numels):
        rec = TensorRecord(key=name, name=name, global_shape=tuple(shape), dtype="torch.bfloat16")
        for rank in range(4):
            ov = intersect_ranges(ShardRange(rank * s_src, s_src), ShardRange(cursor, numel))
            if ov is None:
                continue
            key = f"model::{name}@{ov.start - cursor}"
            rec.shards.append(ShardRecord(rank=rank, file=shard_filename(rank), offset=ov.start - cursor,
                                          length=ov.length, key=key))
            cache.add(shard_filename(rank), key, shards[rank][ov.start - rank * s_src : ov.end - rank * s_src])
        records[name] = rec
        cursor += numel
    cpu = None
    if _WITH_CPU:
        # The reference's re-slice of destination shard 0 at W=8 on host copies of the
        # stored intervals it reads (all in source shard 0); its per-element rate is the
        # baseline for both destination widths.
        from oracle.cpu_reference_path import read_pieces_into_shard

        s8 = -(-total // 8)
        host_src = shards[0][:s8].cpu()
        pieces, cur = [], 0
        for (name, shape), numel in zip(shapes, numels):
            ov = intersect_ranges(ShardRange(0, s8), ShardRange(cur, numel))
            if ov is not None:
                pieces.append((ov.start, [host_src[ov.start : ov.end]]))
            cur += numel
        out = torch.empty(s8, dtype=torch.bfloat16)
        cpu = _cpu_line(s8, _cpu_time(lambda: read_pieces_into_shard(out, pieces), 3), "elements/s",
                        f"destination shard 0 of W=8 ({s8} bf16 elements, {len(pieces)} pieces): per piece "
                        "read_tensor_range into a fresh tensor, then a copy into the flat shard; 3 timed runs "
                        "after 1 warm-up")
        del host_src, pieces, out
    for w_dst in (8, 2):
        s_dst = -(-total // w_dst)
        dests = [torch.empty(s_dst, dtype=torch.bfloat16, device=device) for _ in range(w_dst)]
        layouts = []
        for rank in range(w_dst):
            local, items, cur = ShardRange(rank * s_dst, s_dst), [], 0
            for (name, shape), numel in zip(shapes, numels):
                ov = intersect_ranges(local, ShardRange(cur, numel))
                if ov is not None:
                    items.append(PieceLayout(name, tuple(shape), ov.start - cur, ov.length, ov.start - local.start))
                cur += numel
            layouts.append(items)

        def run():
            for dest, items in zip(dests, layouts):
                load_flat_shard(dest, items, records, cache)

        ms = _time_events(run, max(steps, 5), max(warmup, 2))
        _emit("flat-interval reshard: elements/s", "elements/s", total / (ms * 1e-3), ms, max(steps, 5),
              max(warmup, 2), "bf16", f"Llama-3-8B bf16 flat shards, W=4 -> W={w_dst}", 4 * total,
              {"elements": total, "bytes_per_element": 4},
              _secondary_traffic("reshard", [f"one destination shard of {s_dst:,} elements (W={w_dst})"], [w_dst]),
              cpu)
        del dests
        torch.cuda.empty_cache()
    # Re-slices that cast, W=4 -> W=8: the bf16 checkpoint into fp16 shards (read 2 B +
    # write 2 B), then an fp32 save of the same model into float64 shards (read 4 B + write
    # 8 B): ``read_tensor_range``'s ``.to(out.dtype)`` (``checkpoint/reshard.py:290``).
    s8 = -(-total // 8)
    layouts8 = []
    for rank in range(8):
        local, items, cur = ShardRange(rank * s8, s8), [], 0
        for (name, shape), numel in zip(shapes, numels):
            ov = intersect_ranges(local, ShardRange(cur, numel))
            if ov is not None:
                items.append(PieceLayout(name, tuple(shape), ov.start - cur, ov.length, ov.start - local.start))
            cur += numel
        layouts8.append(items)
    dests = [torch.empty(s8, dtype=torch.float16, device=device) for _ in range(8)]

    def run16():
        for dest, items in zip(dests, layouts8):
            load_flat_shard(dest, items, records, cache)

    ms = _time_events(run16, max(steps, 5), max(warmup, 2))
    _emit("flat-interval reshard with a cast, bf16 -> fp16: elements/s", "elements/s", total / (ms * 1e-3), ms,
          max(steps, 5), max(warmup, 2), "bf16->f16", "Llama-3-8B bf16 flat shards, W=4 -> W=8 fp16 shards",
          4 * total, {"elements": total, "bytes_per_element": 4},
          _secondary_traffic("reshard", [f"bf16 -> fp16: one destination shard of {s8:,} elements (W=8)"], [8]))
    del dests, shards, cache
    torch.cuda.empty_cache()
    shards32 = [torch.randn(s_src, device=device, generator=gen) for _ in range(4)]
    records32, cache32, cursor = {}, DeviceShardCache(), 0
    for (name, shape), numel in zip(shapes, numels):
        rec = TensorRecord(key=name, name=name, global_shape=tuple(shape), dtype="torch.float32")
        for rank in range(4):
            ov = intersect_ranges(ShardRange(rank * s_src, s_src), ShardRange(cursor, numel))
            if ov is None:
                continue
            key = f"model::{name}@{ov.start - cursor}"
            rec.shards.append(ShardRecord(rank=rank, file=shard_filename(rank), offset=ov.start - cursor,
                                          length=ov.length, key=key))
            cache32.add(shard_filename(rank), key, shards32[rank][ov.start - rank * s_src : ov.end - rank * s_src])
        records32[name] = rec
        cursor += numel
    dests = [torch.empty(s8, dtype=torch.float64, device=device) for _ in range(8)]

    def run64():
        for dest, items in zip(dests, layouts8):
            load_flat_shard(dest, items, records32, cache32)

    ms = _time_events(run64, max(steps, 5), max(warmup, 2))
    _emit("flat-interval reshard with a cast, fp32 -> fp64: elements/s", "elements/s", total / (ms * 1e-3), ms,
          max(steps, 5), max(warmup, 2), "f32->f64", "Llama-3-8B fp32 flat shards, W=4 -> W=8 float64 shards",
          12 * total, {"elements": total, "bytes_per_element": 12},
          _secondary_traffic("reshard", [f"fp32 -> fp64: one destination shard of {s8:,} elements (W=8)"], [8]))
    del dests, shards32, cache32
    torch.cuda.empty_cache()
    return 0


def bench_scaler(steps: int, warmup: int) -> int:
    """One Llama-3-70B FSDP rank at W=8: 8,819,213,312 fp32 master params, bf16 grads at scale 2^16.

    Clean step with the multipliers deferred (``defer_unscale``, ``defer_clip``): fused
    unscale + inf check + norm (2 B/param) and unscale + clip + AdamW (26 B/param) =
    28 B/param.  Overflowing step: the check pass only (2 B/param), then skip.  Clean steps
    with the reference's placement (the defaults): ``unscale_`` rewrites the gradient and
    sums the squares of the result in the same pass (read and write bf16: 4 B/param), the
    clip rewrites it again (4 B/param) and the update reads it (26 B/param) = 34 B/param;
    with ``clip_in_step`` the update applies the clip and writes the clipped gradient back
    (26 + 2 B) = 32 B/param.  The gradient is restored from a pristine copy before each such
    step, outside the timed events.
    """
    import torch

    from hybrid_training_amd import GradScaler, GradScalerConfig, GroupHandle, OptimizerConfig, ShardedOptimizer

    device = torch.device("cuda", 0)
    n = 8_819_213_312
    gen = torch.Generator(device=device).manual_seed(70)
    param = torch.nn.Parameter(torch.empty(n, device=device))
    param.grad_dtype = None
    grad = torch.empty(n, dtype=torch.bfloat16, device=device)
    for start in range(0, n, 1 << 30):
        stop = min(n, start + (1 << 30))
        param.data[start:stop].normal_(0.0, 0.02, generator=gen)
        grad[start:stop] = torch.randn(stop - start, device=device, generator=gen).mul_(1e-4 * 65536).to(torch.bfloat16)
    opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=3e-4, betas=(0.9, 0.95), weight_decay=0.1),
                           norm_group=GroupHandle.trivial("world"), device=device, defer_clip=True)
    scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=65536.0, growth_interval=10**9),
                        GroupHandle.trivial("world"), device, defer_unscale=True)
    pristine = grad.clone()

    def engine_step():
        param.grad = grad
        scaler.unscale_([param])
        opt.clip_grad_norm(1.0)
        stepped = scaler.step(opt, [param], already_unscaled=True)
        scaler.update(found_non_finite=False)  # keep the scale fixed across timed steps
        opt.zero_grad(set_to_none=True)
        return stepped

    ms = _time_events(engine_step, max(steps, 5), max(warmup, 2))
    _emit("loss-scaled clipped AdamW step (bf16 grads): params/s", "params/s", n / (ms * 1e-3), ms,
          max(steps, 5), max(warmup, 2), "f32", "Llama-3-70B FSDP rank shard at W=8, bf16 grads, scale 2^16",
          28 * n, {"params": n, "bytes_per_param": 28, "skipped": False},
          _secondary_traffic("scaler", ["fused unscale + clip + AdamW", "unscale + check + norm"], [1, 1]))
    bad = torch.randint(0, n, (n // 1000,), device=device, generator=gen)
    grad[bad] = float("inf")
    ms = _time_events(engine_step, max(steps, 5), max(warmup, 2))
    _emit("loss-scaled step with 0.1% inf gradients (skipped): params/s", "params/s", n / (ms * 1e-3), ms,
          max(steps, 5), max(warmup, 2), "bf16", "Llama-3-70B FSDP rank shard at W=8, bf16 grads, 0.1% inf",
          2 * n, {"params": n, "bytes_per_param": 2, "skipped": True},
          _secondary_traffic("scaler", ["unscale + check + norm"], [1]), _scaler_cpu_baseline() if _WITH_CPU else None)
    # The reference's placement: eager unscale_, then the clip (in place on .grad by
    # default, or fused into the update with clip_in_step), then the update.
    del opt, scaler
    torch.cuda.empty_cache()
    stream = torch.cuda.current_stream(device)
    placements = [
        (False, 34, "loss-scaled clipped AdamW step, reference placement (eager unscale_, eager in-place clip): params/s",
         "defer_unscale=False, defer_clip=False", ["reference placement: eager unscale_ with its overflow check, one pass",
                                                  "reference placement: fold of the piece sums",
                                                  "reference placement: eager in-place clip of .grad",
                                                  "reference placement: AdamW of the clipped gradient"], [1, 1, 1, 1]),
        (True, 32, "loss-scaled clipped AdamW step, reference placement with the clip in the update: params/s",
         "defer_unscale=False, clip_in_step=True", ["reference placement: eager unscale_ with its overflow check, one pass",
                                                   "reference placement: fold of the piece sums",
                                                   "clip_in_step: clip + AdamW, clipped g written back"], [1, 1, 1]),
    ]
    for in_step, per_param, metric, label, traffic_labels, launches in placements:
        opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=3e-4, betas=(0.9, 0.95), weight_decay=0.1),
                               norm_group=GroupHandle.trivial("world"), device=device, clip_in_step=in_step)
        scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=65536.0, growth_interval=10**9),
                            GroupHandle.trivial("world"), device)

        def eager_step(events=None):
            grad.copy_(pristine)  # the next backward's gradient (outside the timed events)
            if events is not None:
                events[0].record(stream)
            param.grad = grad
            scaler.unscale_([param])
            opt.clip_grad_norm(1.0)
            scaler.step(opt, [param], already_unscaled=True)
            scaler.update(found_non_finite=False)
            if events is not None:
                events[1].record(stream)
            opt.zero_grad(set_to_none=True)

        eager_steps, eager_warmup = max(steps, 5), max(warmup, 2)
        for _ in range(eager_warmup):
            eager_step()
        events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(eager_steps)]
        for e in events:
            eager_step(e)
        torch.cuda.synchronize()
        ms = sum(e[0].elapsed_time(e[1]) for e in events) / eager_steps
        if bool(torch.equal(grad[:4096], pristine[:4096])):  # the reference's in-place ops rewrite .grad
            raise RuntimeError("the eager unscale and clip left .grad unchanged")
        _emit(metric, "params/s", n / (ms * 1e-3), ms, eager_steps, eager_warmup, "f32",
              f"Llama-3-70B FSDP rank shard at W=8, bf16 grads, scale 2^16, {label}",
              per_param * n, {"params": n, "bytes_per_param": per_param, "skipped": False},
              _secondary_traffic("scaler", traffic_labels, launches))
        del opt, scaler
    return 0


def _scaler_cpu_baseline() -> dict:
    """The reference's skipped step on the host: ``unscale_`` (bf16 ``grad.mul_``) and the
    finiteness scan, on 2^26 bf16 gradient elements with 0.1% inf.  The clean step has no
    CPU counterpart: torch's CPU AdamW refuses bf16 gradients on fp32 parameters."""
    import torch

    from oracle.cpu_reference_path import unscale_and_check

    n = 1 << 26
    gen = torch.Generator().manual_seed(7)
    grad = (torch.randn(n, generator=gen) * (1e-3 * 65536.0)).to(torch.bfloat16)
    grad[torch.randint(0, n, (n // 1000,), generator=gen)] = float("inf")
    seconds = _cpu_time(lambda: unscale_and_check([grad], 65536.0), 3)
    return _cpu_line(n, seconds, "params/s", f"{n} bf16 gradient elements, 0.1% inf: grad.mul_(2^-16) + "
                     "torch.isfinite scan, 3 timed runs after 1 warm-up")


def _fsdp_cpu_baselines(named, world: int) -> dict:
    """The reference's FSDP op sequences timed on this host (bounded samples).

    pack: one rank's ``_build_shard`` on the embedding and the first transformer block
    (the reference builds the whole padded flat buffer for every rank, so one host
    building all ``world`` shards takes ``world`` times one rank's build); unpack and
    gather on the same parameters.  share, tail, no_sync, no_sync end: rank 0's share of
    2^26 elements per rank."""
    import torch

    from oracle.cpu_reference_path import ReferenceCpuStep, build_shard, full_tensors, gather_full, local_share

    out = {}
    subset = [p.detach().cpu() for name, p in named if name.startswith(("model.embed_tokens.", "model.layers.0."))]
    n_sub = sum(p.numel() for p in subset)
    shard = -(-n_sub // world)
    seconds = _cpu_time(lambda: build_shard(subset, shard * world, shard, 0, torch.float32), 2)
    out["pack"] = _cpu_line(n_sub, seconds * world, "params/s",
                            f"_build_shard of rank 0 over {n_sub} bf16 params (embedding + block 0), 2 timed runs "
                            f"after 1 warm-up; value = params / ({world} x one rank's build)")
    flat = torch.zeros(shard * world, dtype=torch.float32)
    entries, offset = [], 0
    for p in subset:
        flat[offset : offset + p.numel()].copy_(p.reshape(-1))
        entries.append((offset, tuple(p.shape)))
        offset += p.numel()
    del subset
    shards = [s.clone() for s in flat.split(shard)]
    del flat
    out["unpack"] = _cpu_line(n_sub, _cpu_time(lambda: full_tensors(shards, entries), 2), "params/s",
                              f"full_tensors over the same {n_sub} params from {world} fp32 shards: all-gather "
                              "(cat) + a clone per parameter, 2 timed runs after 1 warm-up")
    out["gather"] = _cpu_line(n_sub, _cpu_time(lambda: gather_full(shards, torch.bfloat16), 2), "params/s",
                              f"gather_full over the same {n_sub} params: {world} fp32 shards cast to bf16 and "
                              "placed in the full buffer, 2 timed runs after 1 warm-up")
    del shards
    n = 1 << 26
    gen = torch.Generator().manual_seed(6)
    grads = [torch.randn(n, generator=gen).to(torch.bfloat16) for _ in range(world)]
    rows = [torch.randn(n, generator=gen) for _ in range(world)]
    out["share"] = _cpu_line(n, _cpu_time(lambda: local_share(grads, None, world, torch.float32, torch.float32), 3),
                             "elements/s", f"rank 0's share of {n} elements over {world} bf16 gradients: cast, "
                             "div, rank-order sum, 3 timed runs after 1 warm-up")

    def accumulate():
        for q in range(world):
            rows[q].add_(grads[q].to(torch.float32))

    out["no_sync"] = _cpu_line(world * n, _cpu_time(accumulate, 3), "elements/s",
                               f"{world} x {n} bf16 gradient elements cast and added to fp32 accumulators (add_), "
                               "3 timed runs after 1 warm-up")
    tail = ReferenceCpuStep(n, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)

    def tail_step():
        tail.param.grad = local_share(grads, None, world, torch.float32, torch.float32)
        tail.step(MAX_NORM)

    out["tail"] = _cpu_line(n, _cpu_time(tail_step, 3), "elements/s",
                            f"rank 0's share of {n} elements as above, then the fp64 norm, in-place clip and "
                            "torch.optim.AdamW(foreach=False).step, 3 timed runs after 1 warm-up")
    del tail
    out["no_sync end"] = _cpu_line(n, _cpu_time(lambda: local_share(grads, rows, world, torch.float32,
                                                                     torch.float32), 3), "elements/s",
                                   f"rank 0's share of {n} elements: grad + accumulator for each of {world} ranks, "
                                   "then div and rank-order sum, 3 timed runs after 1 warm-up")
    return out


def bench_fsdp(steps: int, warmup: int) -> int:
    """Llama-3-8B (291 bf16 tensors, 8,030,261,248 params), FSDP at W=8 with fp32 master shards.

    Pack: the 8 ranks' ``FlatParamHandle`` construction (read bf16 2 B + write fp32
    4 B per param).  Unpack: ``full_tensors`` from the 8 shards (read 4 B + write 4 B).
    Gather: ``gather_full``, the all-gather's local side, casting the 8 fp32 shards into
    the padded bf16 compute buffer in one launch (read 4 B + write 2 B).
    Local share: rank 0's ``reduce_scatter_gradient`` over the 8 ranks' padded bf16
    gradients resident on the device (read 8 x 2 B + write 4 B per shard element).
    no_sync: one micro-batch's accumulation of rank 0's slices of the 8 bf16 gradients
    into its fp32 accumulator (read 4 + 2 B, write 4 B per accumulated element).  no_sync
    end: the call after the accumulation, which adds the last micro-batch to the 8
    accumulated rows and reduces them in one pass (read 8 x (4 + 2) B + write 4 B per
    shard element), the first micro-batch set up outside the timed events.
    """
    import torch

    from hybrid_training_amd import FlatParamHandle, FSDPConfig, GroupHandle, MixedPrecisionConfig

    device = torch.device("cuda", 0)
    world = 8
    shapes = _llama3_shapes(32, 4096, 14336, 1024, 128256)
    gen = torch.Generator(device=device).manual_seed(5)
    named = [(name, torch.nn.Parameter(torch.randn(shape, dtype=torch.bfloat16, device=device, generator=gen)))
             for name, shape in shapes]
    total = sum(p.numel() for _, p in named)
    mp = MixedPrecisionConfig(enabled=True, param_dtype="bfloat16", reduce_dtype="float32", master_dtype="float32")
    cpu = _fsdp_cpu_baselines(named, world) if _WITH_CPU else {}

    def build():
        return [FlatParamHandle(named, None, GroupHandle.local_view("shard", world, r), FSDPConfig(), mp, device,
                                keep_originals=True) for r in range(world)]

    handles = []

    def pack():
        handles.clear()
        handles.extend(build())

    ms = _time_events(pack, max(steps, 3), max(warmup, 1))
    shard = handles[0].shard_numel
    _emit("FSDP pack/pad/shard (FlatParamHandle build): params/s", "params/s", total / (ms * 1e-3), ms,
          max(steps, 3), max(warmup, 1), "bf16->f32", f"Llama-3-8B bf16 params -> {world} fp32 master shards",
          6 * total, {"params": total, "world": world, "shard_numel": shard, "bytes_per_param": 6},
          _secondary_traffic("fsdp", ["pack: one rank's fp32 master shard"], [world]), cpu.get("pack"))
    shards = [h.flat_param for h in handles]
    outputs = {}

    def unpack():
        outputs.clear()
        outputs.update(handles[0].full_tensors(peer_shards=shards))

    ms = _time_events(unpack, max(steps, 3), max(warmup, 1))
    _emit("FSDP unpack (full_tensors from all shards): params/s", "params/s", total / (ms * 1e-3), ms,
          max(steps, 3), max(warmup, 1), "f32", f"Llama-3-8B, {world} fp32 shards -> 291 fp32 tensors",
          8 * total, {"params": total, "world": world, "bytes_per_param": 8},
          _secondary_traffic("fsdp", ["unpack: all 291 tensors from 8 shards"], [1]), cpu.get("unpack"))
    outputs.clear()

    def gather():
        handles[0].gather_full(peer_shards=shards)

    ms = _time_events(gather, max(steps, 3), max(warmup, 1))
    _emit("FSDP gather with cast (gather_full: fp32 shards -> bf16 compute buffer): params/s", "params/s",
          total / (ms * 1e-3), ms, max(steps, 3), max(warmup, 1), "f32->bf16",
          f"Llama-3-8B, {world} fp32 master shards -> one padded bf16 compute buffer",
          6 * total, {"params": total, "world": world, "bytes_per_param": 6},
          _secondary_traffic("fsdp", ["gather with cast: 8 fp32 shards into the bf16 compute buffer"], [1]),
          cpu.get("gather"))
    handles[0].reshard()
    del shards
    owner = handles[0]
    handles.clear()
    torch.cuda.empty_cache()
    padded = owner.padded_numel
    grads = [torch.randn(padded, dtype=torch.bfloat16, device=device, generator=gen).mul_(1e-3) for _ in range(world)]

    def share():
        return owner.reduce_scatter_gradient(grads[0], peer_grads=grads)

    ms = _time_events(share, max(steps, 5), max(warmup, 2))
    _emit("FSDP gradient local share (AVG reduce-scatter stand-in): shard elements/s", "elements/s",
          shard / (ms * 1e-3), ms, max(steps, 5), max(warmup, 2), "bf16->f32",
          f"Llama-3-8B rank 0 of W={world}: {world} padded bf16 gradients -> fp32 shard, with norm partials",
          (2 * world + 4) * shard, {"shard_numel": shard, "world": world, "bytes_per_element": 2 * world + 4},
          _secondary_traffic("fsdp", ["gradient local share with norm partials"], [1]), cpu.get("share"))

    # The same share reduced in float64 into a float64 shard (reduce and master dtype
    # float64): read 8 x 2 B + write 8 B per shard element, with float64 norm partials.
    from hybrid_training_amd import _native

    lib = _native.library()
    out64 = torch.empty(shard, dtype=torch.float64, device=device)
    chunk64 = 16384
    partials64 = torch.empty(-(-shard // chunk64), dtype=torch.float64, device=device)
    tiles64 = torch.empty(-(-shard // 256), dtype=torch.float64, device=device)
    grad_ptrs = _native.pointer_array([g.data_ptr() for g in grads])

    def share64():
        _native.check(lib.hbt_grad_local_share_sqnorm(
            grad_ptrs, world, 0, shard, shard, _native.dtype_code(torch.bfloat16), _native.dtype_code(torch.float64),
            float(world), _native.dtype_code(torch.float64), out64.data_ptr(), partials64.data_ptr(),
            tiles64.data_ptr(), _native.stream_of(device)), "bench.local_share_f64")

    ms = _time_events(share64, max(steps, 5), max(warmup, 2))
    _emit("FSDP gradient local share, float64 reduce: shard elements/s", "elements/s", shard / (ms * 1e-3), ms,
          max(steps, 5), max(warmup, 2), "bf16->f64",
          f"Llama-3-8B rank 0 of W={world}: {world} padded bf16 gradients reduced in float64 into a float64 shard, "
          "with norm partials", (2 * world + 8) * shard,
          {"shard_numel": shard, "world": world, "bytes_per_element": 2 * world + 8},
          _secondary_traffic("fsdp", ["float64 reduce: local share with norm partials",
                                      "float64 reduce: tile sums to partials"], [1, 1]))
    del out64, partials64, tiles64

    from hybrid_training_amd import OptimizerConfig, ShardedOptimizer

    opt = ShardedOptimizer([owner.flat_param], OptimizerConfig(learning_rate=LR, betas=BETAS, eps=EPS, weight_decay=WD),
                           norm_group=GroupHandle.local_view("world", world, 0), device=device, defer_clip=True)

    def tail():
        owner.flat_param.grad = owner.reduce_scatter_gradient(grads[0], peer_grads=grads)
        opt.clip_grad_norm(MAX_NORM)
        opt.step()

    ms = _time_events(tail, max(steps, 5), max(warmup, 2))
    _emit("FSDP optimizer tail (local share + clip + AdamW): shard elements/s", "elements/s", shard / (ms * 1e-3),
          ms, max(steps, 5), max(warmup, 2), "bf16->f32",
          f"Llama-3-8B rank 0 of W={world}: local share with norm partials, clip from them, fused AdamW",
          (2 * world + 4 + 28) * shard, {"shard_numel": shard, "world": world, "bytes_per_element": 2 * world + 32},
          _secondary_traffic("fsdp", ["gradient local share with norm partials", "fused clip + AdamW in the tail"],
                             [1, 1]), cpu.get("tail"))

    # no_sync: the first micro-batch copies rank 0's slice of each rank's gradient into
    # the fp32 accumulator (untimed); each timed micro-batch adds the eight slices to it.
    owner.set_accumulate_without_reduction(True)
    owner.reduce_scatter_gradient(grads[0], peer_grads=grads)

    def accumulate():
        owner.reduce_scatter_gradient(grads[0], peer_grads=grads)

    ms = _time_events(accumulate, max(steps, 5), max(warmup, 2))
    _emit("FSDP no_sync gradient accumulation: accumulated elements/s", "elements/s", world * shard / (ms * 1e-3),
          ms, max(steps, 5), max(warmup, 2), "bf16->f32",
          f"Llama-3-8B rank 0 of W={world}: one micro-batch of {world} bf16 gradient slices added to the fp32 "
          "accumulator", 10 * world * shard,
          {"shard_numel": shard, "world": world, "bytes_per_element": 10},
          _secondary_traffic("fsdp", ["no_sync accumulation"], [1]), cpu.get("no_sync"))
    owner.set_accumulate_without_reduction(False)
    owner.flat_param.grad = owner.reduce_scatter_gradient(grads[0], peer_grads=grads)

    stream = torch.cuda.current_stream(device)

    def end_of_accumulation(events=None):
        owner.set_accumulate_without_reduction(True)
        owner.reduce_scatter_gradient(grads[0], peer_grads=grads)  # the first micro-batch, untimed
        owner.set_accumulate_without_reduction(False)
        if events is not None:
            events[0].record(stream)
        owner.flat_param.grad = owner.reduce_scatter_gradient(grads[0], peer_grads=grads)
        if events is not None:
            events[1].record(stream)

    end_steps, end_warmup = max(steps, 5), max(warmup, 2)
    for _ in range(end_warmup):
        end_of_accumulation()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(end_steps)]
    for e in events:
        end_of_accumulation(e)
    torch.cuda.synchronize()
    ms = sum(e[0].elapsed_time(e[1]) for e in events) / end_steps
    _emit("FSDP no_sync end: last micro-batch added and reduced in one pass: shard elements/s", "elements/s",
          shard / (ms * 1e-3), ms, end_steps, end_warmup, "bf16->f32",
          f"Llama-3-8B rank 0 of W={world}: {world} accumulated fp32 rows plus the last micro-batch's bf16 "
          "gradients -> fp32 shard, with norm partials", (6 * world + 4) * shard,
          {"shard_numel": shard, "world": world, "bytes_per_element": 6 * world + 4},
          _secondary_traffic("fsdp", ["no_sync end: accumulate and reduce in one pass"], [1]), cpu.get("no_sync end"))
    del opt, grads, owner, named
    torch.cuda.empty_cache()
    return 0


def _headline_inputs(device, n):
    import torch

    gen = torch.Generator(device=device).manual_seed(0)
    param = torch.nn.Parameter(torch.randn(n, device=device, generator=gen).mul_(0.02))
    grad = torch.randn(n, device=device, generator=torch.Generator(device=device).manual_seed(1)).mul_(1e-4)
    return param, grad


def bench_inplace_clip(steps: int, warmup: int) -> int:
    """The headline shard with the reference's in-place clip (``defer_clip=False``), in the
    two placements the optimizer offers.

    Default (the reference's order): ``clip_grad_norm`` runs the norm pass (read g: 4 B)
    and multiplies ``.grad`` in place (read and write g: 8 B); ``step`` runs the AdamW pass
    on the clipped gradient (read p, g, m, v: 16 B; write p, m, v: 12 B): 40 B/param.
    ``clip_in_step=True``: the update applies the multiplier and writes the clipped
    gradient back in its own pass (read 16 B, write p, g, m, v: 16 B): 36 B/param, with
    ``.grad`` clipped only once ``step`` has run.  Before each step the gradient is
    restored from a pristine copy (standing in for the next backward; not timed), so every
    step clips (norm ~3.17, multiplier ~0.32).  The step time is the HIP event interval from
    the norm pass's launch to the end of the update.
    """
    import torch

    from hybrid_training_amd import GroupHandle, OptimizerConfig, ShardedOptimizer

    device = torch.device("cuda", 0)
    n = SHARD_NUMEL
    param, pristine = _headline_inputs(device, n)
    grad = pristine.clone()
    stream = torch.cuda.current_stream(device)
    runs = [(False, 40, "sharded AdamW + in-place clip step: params/s",
             "norm, clip written to .grad in place, AdamW on the clipped gradient (the reference's order)",
             ["norm pass", "eager in-place clip of .grad", "AdamW of the clipped gradient"], "adamw"),
            (True, 36, "sharded AdamW + in-place clip step, clip applied in the update: params/s",
             "norm, then AdamW applying the clip and writing the clipped gradient back (clip_in_step)",
             ["norm pass", "clip_in_step: clip + AdamW, clipped g written back"], "adamw_write_back")]
    for in_step, per_param, metric, workload, labels, kernel in runs:
        opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=LR, betas=BETAS, eps=EPS, weight_decay=WD),
                               norm_group=GroupHandle.trivial("world"), device=device, defer_clip=False,
                               clip_in_step=in_step)
        param.grad = grad

        def step(events=None):
            grad.copy_(pristine)  # the next backward's gradient (outside the timed events)
            if events is not None:
                events[0].record(stream)
            opt.clip_grad_norm(MAX_NORM)
            if events is not None:
                events[1].record(stream)
            opt.step()
            if events is not None:
                events[2].record(stream)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        if bool(torch.equal(grad[:4096], pristine[:4096])):
            raise RuntimeError("the in-place clip did not leave the clipped gradient in .grad")
        events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        for k in range(steps):
            step(events[k])
        torch.cuda.synchronize()
        clip_ms = sum(e[0].elapsed_time(e[1]) for e in events) / steps
        adamw_ms = sum(e[1].elapsed_time(e[2]) for e in events) / steps
        ms = sum(e[0].elapsed_time(e[2]) for e in events) / steps
        adamw_bytes = (32 if in_step else 28) * n
        adamw_gbps = adamw_bytes / (adamw_ms * 1e-3) / 1e9
        step_gbps = per_param * n / (ms * 1e-3) / 1e9
        log(f"in-place clip ({'in the update' if in_step else 'eager'}): {ms:.3f} ms/step "
            f"(clip_grad_norm {clip_ms:.3f} ms, step {adamw_ms:.3f} ms)")
        line = {
            "metric": metric, "value": n / (ms * 1e-3), "unit": "params/s",
            "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": ms, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (device-generated)",
            "config": {"workload": f"Llama-3-8B FSDP rank shard at W=8: {workload}", "shard_numel": n,
                       "bytes_per_param": per_param},
            "step_hbm_gbps": step_gbps, "step_frac_of_peak": step_gbps / HBM_PEAK_GBPS,
            "kernel_ms": {"clip_grad_norm": clip_ms, kernel: adamw_ms},
            "roofline": {"bound": "hbm", "achieved": adamw_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": adamw_gbps / HBM_PEAK_GBPS,
                         "traffic": _secondary_traffic("inplace_clip", labels[-1:], [1]),
                         "traffic_per": "launch of the dominant kernel"},
            "cpu_baseline": _cpu_step_line(1 << 26, 5) if _WITH_CPU and not in_step else None,
        }
        print(json.dumps(line), flush=True)
        del opt
    return 0


def bench_checkpoint(steps: int, warmup: int) -> int:
    """Llama-3-8B bf16 saved by 4 FSDP ranks to a RAM-backed directory, loaded back at W=8.

    Save: each rank's shard to pinned host memory in one transfer, ``torch.save`` of
    its pieces, SHA-256, manifest, atomic rename.  Load: manifest validation, SHA-256
    verification, ``torch.load(weights_only=True)``, upload, and the device reshard
    into 8 destination shards.  Reported per phase; the device reshard is the part
    this library's kernels do, the rest is host I/O.
    """
    import shutil
    import tempfile

    import torch

    from hybrid_training_amd import (FlatParamHandle, FSDPConfig, GroupHandle, MixedPrecisionConfig,
                                     collect_flat_shard_payload, load_flat_shard_checkpoint, write_checkpoint)

    device = torch.device("cuda", 0)
    shapes = _llama3_shapes(32, 4096, 14336, 1024, 128256)
    gen = torch.Generator(device=device).manual_seed(6)
    named = [(name, torch.nn.Parameter(torch.randint(-16000, 16000, shape, dtype=torch.int16, device=device,
                                                      generator=gen).view(torch.bfloat16)))
             for name, shape in shapes]
    total = sum(p.numel() for _, p in named)
    writers = [FlatParamHandle(named, None, GroupHandle.local_view("shard", 4, r), FSDPConfig(), MixedPrecisionConfig(),
                               device, keep_originals=True) for r in range(4)]
    readers = [FlatParamHandle(named, None, GroupHandle.local_view("shard", 8, r), FSDPConfig(), MixedPrecisionConfig(),
                               device, keep_originals=True) for r in range(8)]
    need = 2 * 2 * total  # the files, with room to spare
    root = None
    if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > need:
        root = "/dev/shm"
    workdir = tempfile.mkdtemp(prefix="hbt-ckpt-", dir=root)
    try:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        shards = [(r, *collect_flat_shard_payload(h, rank=r)) for r, h in enumerate(writers)]
        t1 = time.perf_counter()
        path = write_checkpoint(workdir, 1, shards)
        t2 = time.perf_counter()
        del shards
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t3 = time.perf_counter()
        # One cache for the 8 simulated readers: each file is verified and opened once,
        # as each rank of a real job would open only its own.
        from hybrid_training_amd import CheckpointManifest, ShardFileCache
        from hybrid_training_amd.manifest import MANIFEST_FILENAME

        saved = CheckpointManifest.read(path / MANIFEST_FILENAME)
        shared = ShardFileCache(path, saved, device=device)
        shared.prefetch(sorted(saved.files))  # the ranks of a real job verify their files concurrently
        t_verified = time.perf_counter()
        for r, h in enumerate(readers):
            if r == 0:
                start.record()
            load_flat_shard_checkpoint(path, h, cache=shared)
        stop.record()
        torch.cuda.synchronize()
        t4 = time.perf_counter()
        # the device part of the load on its own: the interval copies from payloads already uploaded
        from hybrid_training_amd import load_flat_shard

        manifest = CheckpointManifest.read(path / MANIFEST_FILENAME)
        cache = ShardFileCache(path, manifest, verify_checksums=False, device=device)
        for f in sorted(manifest.files):
            cache.get(f)
        records = manifest.tensors_by_category("model")
        layouts = [h.local_piece_layout() for h in readers]

        def reshard():
            for h, layout in zip(readers, layouts):
                load_flat_shard(h.flat_param.data, layout, records, cache)

        ms = _time_events(reshard, max(steps, 3), max(warmup, 1))
        size = sum((path / f).stat().st_size for f in manifest.files)
    finally:
        shutil.rmtree(workdir, ignore_errors=True)
    line = {
        "metric": "checkpoint save (W=4) + load with reshard (W=8): seconds", "value": (t2 - t0) + (t4 - t3),
        "unit": "s", "n_gpus": 1, "steps": 1, "warmup": 0, "ms_per_step": ((t2 - t0) + (t4 - t3)) * 1e3,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (device-generated)",
        "config": {"workload": "Llama-3-8B bf16 FSDP checkpoint, W=4 writers -> W=8 readers",
                   "directory": "RAM-backed (/dev/shm)" if root else "the default temporary directory",
                   "elements": total, "file_bytes": size,
                   "phases_s": {"collect_to_pinned_host": t1 - t0, "torch_save_digest_manifest": t2 - t1,
                                "load_verify_upload_reshard": t4 - t3,
                                "of_which_verify_and_open": t_verified - t3},
                   "device_reshard_ms": ms},
        "roofline": {"bound": "hbm", "achieved": 4 * total / (ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": 4 * total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, "traffic": None,
                     "traffic_per": "device reshard of all 8 destination shards"},
    }
    print(json.dumps(line), flush=True)
    return 0


def _link_ceiling(device, nbytes: int = 1 << 30, reps: int = 3) -> dict:
    """Host-link rates of plain pinned-memory copies (GB/s): each direction alone and
    both at once on two streams (per direction), from 32-piece copies of ``nbytes``."""
    import torch

    n = nbytes // 4
    host_down = torch.empty(n, dtype=torch.float32, pin_memory=True)
    host_up = torch.ones(n, dtype=torch.float32, pin_memory=True)
    dev_src = torch.ones(n, dtype=torch.float32, device=device)
    dev_dst = torch.empty(n, dtype=torch.float32, device=device)
    down, up = torch.cuda.Stream(device), torch.cuda.Stream(device)
    pieces = 32

    def copies(stream, dst, src):
        with torch.cuda.stream(stream):
            for a, b in zip(dst.chunk(pieces), src.chunk(pieces)):
                a.copy_(b, non_blocking=True)

    cases = {
        "device_to_host": lambda: copies(down, host_down, dev_src),
        "host_to_device": lambda: copies(up, dev_dst, host_up),
        "duplex_per_direction": lambda: (copies(down, host_down, dev_src), copies(up, dev_dst, host_up)),
    }
    rates = {}
    for name, fn in cases.items():
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        rates[name] = nbytes * reps / (time.perf_counter() - t0) / 1e9
    return rates


def bench_offload(steps: int, warmup: int) -> int:
    """The headline shard with optimizer state offloaded to pinned host memory.

    The device parameter is updated in place; per element the step uploads m and v
    (8 B) and writes back the master parameter, m and v (12 B) over the host link,
    overlapped with the update of neighbouring chunks.  The roofline is the link:
    PCIe 5.0 x16, 64 GB/s per direction, against the 12 B/param write-back direction.
    The line also carries the link's measured rates (``_link_ceiling``, after the timed
    steps): with both directions busy, as in the step, each gets less than alone.  The
    probe runs after the steps because its copy streams, once they have copied, change
    which copy resources the HIP runtime gives streams that copy later (measured: the
    pipeline's streams, copying second in the process, serialised the two directions).
    """
    import torch

    from hybrid_training_amd import GroupHandle, OptimizerConfig, ShardedOptimizer

    device = torch.device("cuda", 0)
    n = SHARD_NUMEL
    param, grad = _headline_inputs(device, n)
    opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=LR, betas=BETAS, eps=EPS, weight_decay=WD,
                                                    cpu_offload_state=True),
                           norm_group=GroupHandle.trivial("world"), device=device, defer_clip=True)
    param.grad = grad

    def step():
        opt.clip_grad_norm(MAX_NORM)
        opt.step()
        param.grad = grad

    steps, warmup = max(1, min(steps, 5)), max(1, min(warmup, 2))
    ms = _time_events(step, steps, warmup)
    link = _link_ceiling(device)
    link_gbps = 12 * n / (ms * 1e-3) / 1e9
    line = {
        "metric": "sharded AdamW+clip step with host-offloaded state: params/s", "value": n / (ms * 1e-3),
        "unit": "params/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (device-generated)",
        "config": {"workload": "Llama-3-8B FSDP rank shard at W=8, AdamW state in pinned host memory",
                   "shard_numel": n, "link_bytes_per_param": {"host_to_device": 8, "device_to_host": 12}},
        "roofline": {"bound": "pcie", "achieved": link_gbps, "peak": 64.0, "unit": "GB/s",
                     "frac": link_gbps / 64.0, "traffic": None, "traffic_per": "step, device-to-host direction"},
        "link_measured_gbps": link,
        "frac_of_measured_duplex": link_gbps / link["duplex_per_direction"],
        # the reference's offload steps the host masters with torch's CPU AdamW
        "cpu_baseline": _cpu_step_line(1 << 26, 5) if _WITH_CPU else None,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_param_offload(steps: int, warmup: int) -> int:
    """The headline shard as an FSDP unit with ``cpu_offload_params``: shard, gradient and
    AdamW state in pinned host memory.

    Per step, as the reference runs it (``fsdp.py:763-764``, then the clip and the
    optimizer step on the host shard): the local share's gradient shard is copied down to
    the host (4 B/param), the clip takes its norm from the local share's partials (no
    read), and the step streams p, g, m, v up (16 B) and p, m, v and the clipped g down
    (16 B), chunk by chunk, overlapped with the update.  The device holds none of the
    shard or its state, only the staging slots.  The roofline is the link's heavier
    direction, device to host: 20 B/param.  The line also gives the step's bound at the
    link rates measured in the same process: the gradient copy alone in one direction
    (it must have landed when the reduce-scatter returns), then the streamed step with
    both directions busy.

    Beside it, the reference's own step for this configuration: torch's CPU AdamW
    (``foreach`` off, its CPU default) on a host shard after the in-place clip, timed on
    a 2^25-element sample with torch's host threads and scaled to the full shard.  The
    link's own rates are measured after the timed steps, for the reason given under
    ``bench_offload``.
    """
    import torch
    import torch.nn as nn

    from hybrid_training_amd import (FlatParamHandle, FSDPConfig, GroupHandle, MixedPrecisionConfig,
                                     OptimizerConfig, ShardedOptimizer)

    device = torch.device("cuda", 0)
    n = SHARD_NUMEL
    param, grad_full = _headline_inputs(device, n)
    handle = FlatParamHandle([("shard", nn.Parameter(param))], None, GroupHandle.trivial("shard"),
                             FSDPConfig(cpu_offload_params=True), MixedPrecisionConfig(), device,
                             keep_originals=True)
    del param
    torch.cuda.empty_cache()
    opt = ShardedOptimizer([handle.flat_param], OptimizerConfig(learning_rate=LR, betas=BETAS, eps=EPS,
                                                                weight_decay=WD),
                           norm_group=GroupHandle.trivial("world"), device=device)

    def step():
        handle.flat_param.grad = handle.reduce_scatter_gradient(grad_full)
        opt.clip_grad_norm(MAX_NORM)
        opt.step()

    steps, warmup = max(1, min(steps, 5)), max(1, min(warmup, 2))
    ms = _time_events(step, steps, warmup)
    link = _link_ceiling(device)
    down, up = 20 * n, 16 * n
    link_gbps = down / (ms * 1e-3) / 1e9

    # the reference's step on the host: clip in place, then torch's CPU AdamW
    sample = 1 << 25
    gen = torch.Generator().manual_seed(0)
    p_cpu = nn.Parameter(torch.randn(sample, generator=gen) * 0.02)
    g_cpu = torch.randn(sample, generator=gen) * 1e-4
    ref = torch.optim.AdamW([p_cpu], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)

    def cpu_step():
        g = g_cpu.clone()
        norm = float(g.double().pow(2).sum().sqrt())
        coef = MAX_NORM / (norm + 1e-6)
        if coef < 1.0:
            g.mul_(coef)
        p_cpu.grad = g
        ref.step()

    cpu_step()
    reps = 3
    start = time.perf_counter()
    for _ in range(reps):
        cpu_step()
    cpu_s = (time.perf_counter() - start) / reps
    cpu_rate = sample / cpu_s
    line = {
        "metric": "FSDP step with the shard offloaded to host memory (gradient down, clip, AdamW): params/s",
        "value": n / (ms * 1e-3), "unit": "params/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (device-generated)",
        "config": {"workload": "Llama-3-8B FSDP rank shard at W=8, cpu_offload_params: shard, gradient and AdamW "
                               "state in pinned host memory",
                   "shard_numel": n, "link_bytes_per_param": {"host_to_device": 16, "device_to_host": 20},
                   "link_bytes_per_step": {"host_to_device": up, "device_to_host": down}},
        "roofline": {"bound": "pcie", "achieved": link_gbps, "peak": 64.0, "unit": "GB/s",
                     "frac": link_gbps / 64.0, "traffic": None, "traffic_per": "step, device-to-host direction"},
        "link_measured_gbps": link,
        "frac_of_measured_duplex": link_gbps / link["duplex_per_direction"],
        "link_bound_ms": (4 * n / link["device_to_host"] + 16 * n / link["duplex_per_direction"]) / 1e6,
        "frac_of_link_bound": (4 * n / link["device_to_host"] + 16 * n / link["duplex_per_direction"]) / 1e6 / ms,
        "cpu_baseline": {"value": cpu_rate, "unit": "params/s", "cores": torch.get_num_threads(), "kind": "port",
                         "sample": f"{sample} fp32 elements, mean of {reps} steps: torch CPU AdamW (foreach off) "
                                   "after the in-place clip, the reference's step on an offloaded shard",
                         "ms_per_step": cpu_s * 1e3, "ms_per_step_at_shard": n / cpu_rate * 1e3},
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_sgd(steps: int, warmup: int) -> int:
    """The headline shard with the reference's other inner optimizer: SGD, momentum 0.9.

    Norm pass (4 B) + fused clip + SGD with a momentum buffer (read p, g, buf; write
    p, buf: 20 B) = 24 B/param.
    """
    import torch

    from hybrid_training_amd import GroupHandle, OptimizerConfig, ShardedOptimizer

    device = torch.device("cuda", 0)
    n = SHARD_NUMEL
    param, grad = _headline_inputs(device, n)
    opt = ShardedOptimizer([param], OptimizerConfig(name="sgd", learning_rate=LR, momentum=0.9, weight_decay=WD),
                           norm_group=GroupHandle.trivial("world"), device=device, defer_clip=True)
    param.grad = grad

    def step():
        opt.clip_grad_norm(MAX_NORM)
        opt.step()
        param.grad = grad

    ms = _time_events(step, steps, warmup)
    _emit("sharded SGD(momentum 0.9)+clip step: params/s", "params/s", n / (ms * 1e-3), ms, steps, warmup, "f32",
          "Llama-3-8B FSDP rank shard at W=8: global-norm clip + SGD with momentum", 24 * n,
          {"shard_numel": n, "bytes_per_param": 24},
          _secondary_traffic("sgd", ["SGD with momentum (20 B/param)", "norm pass"], [1, 1]),
          _cpu_step_line(1 << 26, 5, momentum=0.9) if _WITH_CPU else None)
    return 0


def bench_lowp(steps: int, warmup: int) -> int:
    """The headline shard with bf16 masters: a bf16 model with mixed precision off keeps its
    parameters, gradients and optimizer state in bf16 (``parallel/fsdp.py:379-393``).

    AdamW: norm pass (read g: 2 B) + fused clip + AdamW (read p, g, m, v: 8 B; write p, m,
    v: 6 B) = 16 B/param.  SGD with momentum 0.9: norm pass (2 B) + fused clip + SGD (read
    p, g, buf: 6 B; write p, buf: 4 B) = 12 B/param.
    """
    import torch

    from hybrid_training_amd import GroupHandle, OptimizerConfig, ShardedOptimizer

    device = torch.device("cuda", 0)
    n = SHARD_NUMEL
    gen = torch.Generator(device=device).manual_seed(12)
    param = torch.nn.Parameter(torch.empty(n, dtype=torch.bfloat16, device=device))
    grad = torch.empty(n, dtype=torch.bfloat16, device=device)
    for start in range(0, n, 1 << 28):
        stop = min(n, start + (1 << 28))
        param.data[start:stop] = torch.randn(stop - start, device=device, generator=gen).mul_(0.02).to(torch.bfloat16)
        grad[start:stop] = torch.randn(stop - start, device=device, generator=gen).mul_(1e-4).to(torch.bfloat16)
    runs = [("adamw", OptimizerConfig(learning_rate=LR, betas=BETAS, eps=EPS, weight_decay=WD), 16, None,
             "sharded AdamW+clip step, bf16 masters: params/s", ["bf16 masters: fused clip + AdamW", "norm pass"]),
            ("sgd", OptimizerConfig(name="sgd", learning_rate=LR, momentum=0.9, weight_decay=WD), 12, 0.9,
             "sharded SGD(momentum 0.9)+clip step, bf16 masters: params/s",
             ["bf16 masters: fused clip + SGD with momentum", "norm pass"])]
    for name, config, per_param, momentum, metric, labels in runs:
        opt = ShardedOptimizer([param], config, norm_group=GroupHandle.trivial("world"), device=device, defer_clip=True)
        param.grad = grad

        def step():
            opt.clip_grad_norm(MAX_NORM)
            opt.step()
            param.grad = grad

        ms = _time_events(step, steps, warmup)
        _emit(metric, "params/s", n / (ms * 1e-3), ms, steps, warmup, "bf16",
              f"Llama-3-8B FSDP rank shard at W=8, bf16 parameters, gradients and {name} state", per_param * n,
              {"shard_numel": n, "bytes_per_param": per_param},
              _secondary_traffic("lowp", labels, [1, 1]),
              _cpu_step_line(1 << 26, 3, momentum=momentum, dtype=torch.bfloat16) if _WITH_CPU else None)
        del opt
        param.grad = None
        torch.cuda.empty_cache()
    return 0


def bench_mlp(steps: int, warmup: int) -> int:
    """The reference's CPU-runnable case on the device: the MLP Linear(23,32)-ReLU-Linear(32,32)-
    ReLU-Linear(32,1) (1,857 fp32 parameters) as FSDP units at W=2 (shards of 929, pad 1) and
    W=4 (465, pad 3), all ranks on one GPU.  Per rank and step, the drop-in tail: the local
    share of the ranks' padded gradients (the AVG reduce-scatter's arithmetic, with norm
    partials), the clip from those partials and the fused AdamW (lr 1e-3, wd 0.01) on the
    flat shard.  Microseconds per rank-step at this size measure launch cost, not HBM.
    Each W is timed eagerly and then replayed from one HIP graph recording of all ranks'
    tails (``StepGraph``).
    """
    import torch

    from hybrid_training_amd import (FlatParamHandle, FSDPConfig, GroupHandle, MixedPrecisionConfig,
                                     OptimizerConfig, ShardedOptimizer, StepGraph)

    device = torch.device("cuda", 0)
    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(23, 32), torch.nn.ReLU(), torch.nn.Linear(32, 32), torch.nn.ReLU(),
                                torch.nn.Linear(32, 1)).to(device)
    named = list(model.named_parameters())
    mp = MixedPrecisionConfig(enabled=False)
    # A step takes tens of microseconds: at least 500 timed steps (under 0.2 s) keep the
    # launch-time jitter out of the mean.
    mlp_steps, mlp_warmup = max(steps, 500), max(warmup, 50)
    for world in (2, 4):
        handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", world, r), FSDPConfig(), mp, device,
                                   keep_originals=True) for r in range(world)]
        padded, shard = handles[0].padded_numel, handles[0].shard_numel
        gen = torch.Generator(device=device).manual_seed(world)
        grads = [torch.randn(padded, device=device, generator=gen) for _ in range(world)]
        for g in grads:
            g[1857:] = 0.0  # the padding carries no gradient
        opts = [ShardedOptimizer([h.flat_param], OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                                 norm_group=GroupHandle.local_view("world", world, r), device=device, defer_clip=True)
                for r, h in enumerate(handles)]

        def tail():
            for r, (h, opt) in enumerate(zip(handles, opts)):
                h.flat_param.grad = h.reduce_scatter_gradient(grads[r], peer_grads=grads)
                opt.clip_grad_norm(1.0)
                opt.step()

        ms = _time_events(tail, mlp_steps, mlp_warmup)
        cpu = None
        if _WITH_CPU:
            from oracle.cpu_reference_path import ReferenceMlpTail

            ref = ReferenceMlpTail([g.cpu() for g in grads], shard, lr=1e-3, weight_decay=0.01)
            seconds = _cpu_time(lambda: ref.step(1.0), 200)
            cpu = _cpu_line(world, seconds, "rank-steps/s",
                            f"the {world}-rank tail on {shard}-element shards: local shares, fp64 norm, clip, "
                            "torch.optim.AdamW(foreach=False) per rank (tensors this small run on one thread); "
                            "200 timed steps after 1 warm-up")
        per_rank_us = ms * 1e3 / world
        _emit(f"FSDP MLP drop-in tail at W={world} (local share + clip + AdamW): rank-steps/s", "rank-steps/s",
              world / (ms * 1e-3), ms, mlp_steps, mlp_warmup, "f32",
              f"MLP 23-32-32-1 (1,857 fp32 params), FSDP W={world}: shards of {shard}, all ranks on one GPU",
              world * shard * (4 * world + 4 + 28),
              {"params": 1857, "world": world, "shard_numel": shard, "us_per_rank_step": per_rank_us},
              None, cpu)
        # The same tail recorded once into a HIP graph: each replay rewrites the
        # optimizers' step scalars from their host state, then runs every rank's
        # launches with one graph launch.
        graph = StepGraph(tail)
        ms = _time_events(graph.replay, mlp_steps, mlp_warmup)
        _emit(f"FSDP MLP drop-in tail at W={world}, replayed from one HIP graph: rank-steps/s", "rank-steps/s",
              world / (ms * 1e-3), ms, mlp_steps, mlp_warmup, "f32",
              f"MLP 23-32-32-1 (1,857 fp32 params), FSDP W={world}: the tail of all {world} ranks recorded "
              "into one HIP graph (StepGraph) and replayed", world * shard * (4 * world + 4 + 28),
              {"params": 1857, "world": world, "shard_numel": shard, "us_per_rank_step": ms * 1e3 / world},
              None, cpu)
        del graph, handles, opts, grads
    return 0


def bench_torch_adamw(steps: int, warmup: int) -> int:
    """Stock PyTorch on the same GPU and shard: clip_grad_norm_ (foreach) + AdamW(fused=True).

    A comparison point, not this library: the same step written with torch's own GPU
    kernels.  Algorithmic bytes as for the fused path with an in-place clip (40 B/param).
    """
    import torch

    device = torch.device("cuda", 0)
    n = SHARD_NUMEL
    param, grad = _headline_inputs(device, n)
    opt = torch.optim.AdamW([param], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, fused=True)
    param.grad = grad

    def step():
        torch.nn.utils.clip_grad_norm_([param], MAX_NORM, foreach=True)
        opt.step()

    ms = _time_events(step, steps, warmup)
    _emit("torch clip_grad_norm_ + AdamW(fused=True) step: params/s", "params/s", n / (ms * 1e-3), ms, steps,
          warmup, "f32", "Llama-3-8B FSDP rank shard at W=8, stock PyTorch-ROCm kernels (comparison)", 40 * n,
          {"shard_numel": n, "bytes_per_param": 40, "torch": torch.__version__})
    return 0


def bench_copy_ceiling(steps: int, warmup: int) -> int:
    """The copy ceilings: torch's device-to-device ``copy_`` (a hipMemcpy blit) against the
    library's interval copy, one fp32 record of 1 GiB and of 16 GiB (8 B per element moved)."""
    import torch

    from hybrid_training_amd import _native

    device = torch.device("cuda", 0)
    big = 1 << 32
    src = torch.ones(big, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for n in (1 << 28, big):
        plan = _native.CopyPlan(device)
        plan.add(src, 0, dst, 0, n)
        ms_lib = _time_events(lambda: plan.run(src_dtype=torch.float32, dst_dtype=torch.float32), steps, warmup)
        ms_torch = _time_events(lambda: dst[:n].copy_(src[:n]), steps, warmup)
        for name, ms in (("hbt_copy_intervals (aligned kernel)", ms_lib), ("torch copy_ (hipMemcpy D2D)", ms_torch)):
            _emit(f"fp32 copy ceiling, {name}: GB/s", "GB/s", 8 * n / (ms * 1e-3) / 1e9, ms, steps, warmup, "f32",
                  f"one {4 * n / 2**30:.0f} GiB fp32 buffer copied to another", 8 * n, {"elements": n})
    return 0


SECONDARY = {"buckets": bench_buckets, "reshard": bench_reshard, "scaler": bench_scaler, "fsdp": bench_fsdp,
             "inplace_clip": bench_inplace_clip, "torch_adamw": bench_torch_adamw, "sgd": bench_sgd,
             "offload": bench_offload, "param_offload": bench_param_offload, "checkpoint": bench_checkpoint, "copy_ceiling": bench_copy_ceiling,
             "lowp": bench_lowp, "mlp": bench_mlp}


if __name__ == "__main__":
    sys.exit(main())
