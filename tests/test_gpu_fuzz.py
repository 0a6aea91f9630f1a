"""Seeded random configurations through the flat-parameter, checkpoint and DDP paths (GPU).

Each case draws a parameter list (odd sizes, empty tensors and multiples of 256 mixed,
so plans take both the aligned and the general copy kernel), a group size, parameter
and gradient dtypes and a reduce dtype, then checks every rank bitwise against the
oracle: the packed shard (``parallel/fsdp.py:434-454``), the gathered tensors
(``:912-925``), the gradient local share (``:704-781``) and a two-micro-batch
``no_sync`` reduction (``:733-749``).  Random checkpoint reshards and DDP bucket packs
follow, each against the global vector or torch's own CPU arithmetic, and random AdamW
and SGD runs with the global-norm clip and loss-scaled runs with injected overflows
against the oracle; offloaded runs against the in-HBM path; weighted norms against a
brute-force fp64 sum; checkpoints saved and reloaded at random widths through the format
on disk; and random optimizer steps replayed from a HIP graph recording against the same
steps taken eagerly.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import FlatParamHandle, FSDPConfig, GroupHandle, MixedPrecisionConfig

pytestmark = pytest.mark.gpu

_NAMES = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16",
          torch.float64: "float64"}


def _host_bits(t: torch.Tensor) -> np.ndarray:
    """A host copy in the oracle's storage: float32 values, or uint16 bit patterns of a
    2-byte dtype (compared with np.array_equal, so bits, signed zeros included)."""
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def _shapes(rng: np.random.Generator) -> list[tuple[int, ...]]:
    shapes = []
    for _ in range(int(rng.integers(1, 12))):
        kind = int(rng.integers(0, 4))
        if kind == 0:
            shapes.append((int(rng.integers(0, 3)),))                     # empty or tiny
        elif kind == 1:
            shapes.append((int(rng.integers(1, 9)) * 256,))                # whole chunks
        elif kind == 2:
            shapes.append((int(rng.integers(1, 40)), int(rng.integers(1, 70))))
        else:
            shapes.append((int(rng.integers(1, 5000)),))
    if all(int(np.prod(s)) == 0 for s in shapes):
        shapes.append((3,))
    return shapes


def _fsdp_case(device, case: int, groups: tuple[int, ...] | None = None) -> None:
    """One random FSDP configuration; ``groups``: the group sizes to draw from (default 1-9)."""
    rng = np.random.default_rng(1000 + case)
    shapes = _shapes(rng)
    group = int(rng.integers(1, 10)) if groups is None else int(rng.choice(groups))
    param_dtype = [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
    grad_dtype = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    reduce = [torch.float32, torch.bfloat16, torch.float16, torch.float64][int(rng.integers(0, 4))]
    gen = torch.Generator(device=device).manual_seed(case)
    named = [(f"p{i}", torch.nn.Parameter(torch.randn(s, device=device, generator=gen).to(param_dtype)))
             for i, s in enumerate(shapes)]
    mp = MixedPrecisionConfig(enabled=True, param_dtype="bfloat16", reduce_dtype=_NAMES[reduce],
                              master_dtype="float32")
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(), mp, device,
                               keep_originals=True) for r in range(group)]
    host = [p.detach().float().cpu().numpy() for _, p in named]   # exact widening of bf16
    total = sum(int(np.prod(s)) for s in shapes)
    shard, padded, _ = oracle.even_shards(total, group)
    context = f"case {case}: shapes {shapes}, G={group}, {param_dtype} params, {grad_dtype} grads, reduce {reduce}"
    for rank, h in enumerate(handles):
        assert (h.total_numel, h.shard_numel, h.padded_numel) == (total, shard, padded), context
        expect = oracle.pack_shard(host, group, rank)
        assert np.array_equal(h.flat_param.detach().cpu().numpy().view(np.int32), expect.view(np.int32)), context
    full = handles[0].full_tensors(peer_shards=[h.flat_param for h in handles])
    for (name, p), values in zip(named, host):
        assert full[name].shape == p.shape, context
        assert np.array_equal(full[name].float().cpu().numpy().view(np.int32), values.view(np.int32)), context
    grads = [[(torch.randn(padded, device=device, generator=gen) * 0.5).to(grad_dtype) for _ in range(group)]
             for _ in range(2)]
    divisor = float(group) if group > 1 else 1.0
    for rank, h in enumerate(handles):
        valid = max(0, min(shard, total - rank * shard))
        peers = grads[1] if group > 1 else None
        out = h.reduce_scatter_gradient(grads[1][rank], peer_grads=peers)
        expect = oracle.local_share([g.float().cpu().numpy() for g in grads[1]], rank, shard, valid, divisor,
                                    _NAMES[reduce])
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32)), (context, rank)
        h.set_accumulate_without_reduction(True)
        assert h.reduce_scatter_gradient(grads[0][rank], peer_grads=grads[0] if group > 1 else None) is None
        h.set_accumulate_without_reduction(False)
        out = h.reduce_scatter_gradient(grads[1][rank], peer_grads=peers)
        totals = [oracle.no_sync_accumulate([grads[m][q].float().cpu().numpy() for m in range(2)], _NAMES[reduce])
                  for q in range(group)]
        expect = oracle.local_share(totals, rank, shard, valid, divisor, _NAMES[reduce])
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32)), (context, rank)


@pytest.mark.parametrize("case", range(120))
def test_random_fsdp_configurations(device, case):
    """Seeded FSDP configurations with 1-9 ranks: every rank's shard, the gathered
    tensors, the local share and a two-micro-batch ``no_sync`` reduction bitwise the
    oracle's."""
    _fsdp_case(device, case)


@pytest.mark.parametrize("case", range(12))
def test_random_large_group_fsdp_configurations(device, case):
    """The same configurations with 16 to 64 ranks (``HBT_MAX_LOCAL_RANKS``), the run-time
    group-size kernels throughout."""
    _fsdp_case(device, 7000 + case, (16, 31, 32, 33, 63, 64))


@pytest.mark.parametrize("case", range(40))
def test_random_fsdp_units_without_mixed_precision(device, case):
    """Mixed precision off (``parallel/fsdp.py:379-392``): the master, compute and reduce
    dtypes are the parameters' own, fp32, bf16 or fp16.  Every rank's shard packs bitwise in
    that dtype, the gathered tensors come back bitwise, the local share and a two-micro-batch
    ``no_sync`` reduction are the oracle's in that dtype, and one clipped AdamW step on each
    rank's shard, with the norm taken from the local share's partials, is the oracle's."""
    from hybrid_training_amd import OptimizerConfig, ShardedOptimizer

    rng = np.random.default_rng(9000 + case)
    shapes = _shapes(rng)
    group = int(rng.integers(1, 10))
    dtype = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    dt = _NAMES[dtype]
    gen = torch.Generator(device=device).manual_seed(case)
    named = [(f"p{i}", torch.nn.Parameter((torch.randn(s, device=device, generator=gen) * 0.1).to(dtype)))
             for i, s in enumerate(shapes)]
    mp = MixedPrecisionConfig(enabled=False)
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(), mp, device,
                               keep_originals=True) for r in range(group)]
    host = [p.detach().float().cpu().numpy() for _, p in named]   # exact widening
    total = sum(int(np.prod(s)) for s in shapes)
    shard, padded, _ = oracle.even_shards(total, group)
    context = f"case {case}: shapes {shapes}, G={group}, {dt} without mixed precision"
    for rank, h in enumerate(handles):
        assert h.flat_param.dtype == dtype, context
        expect = oracle.to_bits(oracle.pack_shard(host, group, rank), dt)
        assert np.array_equal(_host_bits(h.flat_param), expect), (context, rank)
    full = handles[0].full_tensors(peer_shards=[h.flat_param for h in handles])
    for (name, p), values in zip(named, host):
        assert full[name].dtype == dtype and full[name].shape == p.shape, context
        assert np.array_equal(_host_bits(full[name]), oracle.to_bits(values, dt).reshape(p.shape)), context
    grads = [[(torch.randn(padded, device=device, generator=gen) * 0.05).to(dtype) for _ in range(group)]
             for _ in range(2)]
    for g in grads[0] + grads[1]:
        g[total:] = 0.0
    divisor = float(group) if group > 1 else 1.0
    wide = [[g.float().cpu().numpy() for g in micro] for micro in grads]
    for rank, h in enumerate(handles):
        valid = max(0, min(shard, total - rank * shard))
        peers = grads[1] if group > 1 else None
        out = h.reduce_scatter_gradient(grads[1][rank], peer_grads=peers)
        share = oracle.to_bits(oracle.local_share(wide[1], rank, shard, valid, divisor, dt), dt)
        assert out.dtype == dtype and np.array_equal(_host_bits(out), share), (context, rank)
        # one clipped AdamW step on this rank's shard; the norm comes from the share's partials
        param = h.flat_param
        param.grad = out
        opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=1e-3, betas=(0.9, 0.999), eps=1e-3,
                                                        weight_decay=0.01),
                               norm_group=GroupHandle.local_view("world", group, rank), device=device)
        P = _host_bits(param)
        norm = float(opt.clip_grad_norm(0.01))
        mul = oracle.clip_multiplier(norm, 0.01)
        sq = oracle.sqnorm(share, dtype=dt)
        assert abs(norm - sq ** 0.5) <= 1e-9 * max(norm, 1e-30), (context, rank)
        opt.step()
        sc = oracle.adamw_scalars(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-3, weight_decay=0.01, step=1.0)
        clipped = np.empty_like(share)
        oracle.adamw_step(P, share.copy(), np.zeros_like(P), np.zeros_like(P), sc, grad_mul=mul, dtype=dt,
                          grad_out=clipped)
        assert np.array_equal(_host_bits(param), P), (context, rank)
        assert np.array_equal(_host_bits(param.grad), clipped), (context, rank)
        # no_sync: the first micro-batch accumulates, the second reduces the sums
        h.set_accumulate_without_reduction(True)
        assert h.reduce_scatter_gradient(grads[0][rank], peer_grads=grads[0] if group > 1 else None) is None
        h.set_accumulate_without_reduction(False)
        out = h.reduce_scatter_gradient(grads[1][rank], peer_grads=peers)
        totals = [oracle.no_sync_accumulate([wide[m][q] for m in range(2)], dt) for q in range(group)]
        expect = oracle.to_bits(oracle.local_share(totals, rank, shard, valid, divisor, dt), dt)
        assert np.array_equal(_host_bits(out), expect), (context, rank)


@pytest.mark.parametrize("case", range(60))
def test_random_checkpoint_reshards(device, case):
    """Random layouts saved by 1-5 writers (fp64, fp32, bf16 or fp16) as per-tensor shard
    records and loaded by 1-6 readers into any of those dtypes (``checkpoint/reshard.py:200-305``,
    ``:290``; ``checkpoint/reader.py:328-351``): every reader's shard is the matching slice of the
    global flat vector, cast to the destination dtype as torch's ``Tensor.to`` casts it, and
    its padding tail is left untouched."""
    from hybrid_training_amd import load_flat_shard

    from .test_gpu_reshard import _layout, _save

    rng = np.random.default_rng(5000 + case)
    shapes = _shapes(rng)
    named = [(f"p{i}", s) for i, s in enumerate(shapes)]
    dtypes = [torch.float64, torch.float32, torch.bfloat16, torch.float16]
    src_dtype = dtypes[int(rng.integers(0, 4))]
    dst_dtype = dtypes[int(rng.integers(0, 4))]
    writers, readers = int(rng.integers(1, 6)), int(rng.integers(1, 7))
    total = sum(int(np.prod(s)) for s in shapes)
    gen = torch.Generator(device=device).manual_seed(case)
    flat = torch.randn(total, device=device, generator=gen).to(src_dtype)
    s_src, padded_src, _ = oracle.even_shards(total, writers)
    padded = torch.zeros(padded_src, dtype=src_dtype, device=device)
    padded[:total] = flat
    shards = [padded[r * s_src:(r + 1) * s_src].clone() for r in range(writers)]
    records, cache = _save(named, shards, s_src, str(src_dtype))
    expect_flat = flat.cpu().to(dst_dtype)
    s_dst, _, _ = oracle.even_shards(total, readers)
    context = f"case {case}: shapes {shapes}, {writers} -> {readers}, {src_dtype} -> {dst_dtype}"
    for rank in range(readers):
        dest = torch.full((s_dst,), 7.0, device=device).to(dst_dtype)
        load_flat_shard(dest, _layout(named, rank, s_dst), records, cache)
        valid = max(0, min(s_dst, total - rank * s_dst))
        got = dest.cpu()
        assert torch.equal(got[:valid], expect_flat[rank * s_dst:rank * s_dst + valid]), (context, rank)
        assert bool((got[valid:] == 7.0).all()), (context, rank)


@pytest.mark.parametrize("case", range(60))
def test_random_ddp_bucket_packs(device, case):
    """Random fp32/bf16/fp16 parameter lists, bucket caps and world sizes, with unused
    parameters (``parallel/ddp.py:397-463``, ``:479-523``, ``:579-640``): every gradient
    comes back as its bucket view holding ``grad / W`` rounded to its dtype, as torch's
    CPU ``div`` gives, and an unused parameter's view holds zeros."""
    from hybrid_training_amd import BucketedGradients, DDPConfig

    rng = np.random.default_rng(9000 + case)
    shapes = _shapes(rng)
    world = int(rng.integers(1, 9))
    cap_mb = float(rng.choice([1e-5, 1e-3, 0.01, 25.0]))
    gen = torch.Generator(device=device).manual_seed(case)
    named, expect = [], {}
    for i, s in enumerate(shapes):
        dtype = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
        p = torch.nn.Parameter(torch.empty(s, device=device, dtype=dtype))
        if rng.random() < 0.15:
            expect[f"p{i}"] = torch.zeros(s, dtype=dtype)
        else:
            p.grad = torch.randn(s, device=device, generator=gen).to(dtype)
            g = p.grad.detach().cpu()
            expect[f"p{i}"] = g.div(world) if world > 1 else g
        named.append((f"p{i}", p))
    group = GroupHandle.local_view("data_parallel", world, 0) if world > 1 else GroupHandle.trivial()
    ddp = BucketedGradients(named, group, DDPConfig(bucket_cap_mb=cap_mb, find_unused_parameters=True))
    ddp.synchronize()
    context = f"case {case}: shapes {shapes}, W={world}, cap {cap_mb} MB"
    for name, p in named:
        got = p.grad.detach().cpu()
        assert got.dtype == expect[name].dtype and got.shape == expect[name].shape, (context, name)
        bits = torch.int16 if got.element_size() == 2 else torch.int32
        assert torch.equal(got.contiguous().view(bits), expect[name].contiguous().view(bits)), (context, name)


@pytest.mark.parametrize("case", range(40))
def test_random_adamw_clip_steps(device, case):
    """Random parameter lists (up to 40 tensors, so launches split at 16, empty ones
    included), master dtypes (fp32, bf16, fp16), hyperparameters (both branches of torch's
    lerp), clip thresholds and deferred or in-place clipping, two steps of
    ``clip_grad_norm`` + ``step`` (``optim/sharded_optimizer.py:310-355``): parameters and
    state bitwise the oracle's AdamW with the clip multiplier formed from the returned
    norm, and ``.grad`` after the step the oracle's clipped gradient (in place) or the
    untouched one (deferred)."""
    from hybrid_training_amd import OptimizerConfig, ShardedOptimizer

    rng = np.random.default_rng(7000 + case)
    sizes = [int(rng.choice([0, 1, 7, 256, 1000, 4097])) if rng.random() < 0.3 else int(rng.integers(1, 20000))
             for _ in range(int(rng.integers(1, 41)))]
    lr = float(rng.choice([1e-4, 3e-4, 1e-3]))
    betas = [(0.9, 0.95), (0.8, 0.999), (0.4, 0.9)][int(rng.integers(0, 3))]
    wd = float(rng.choice([0.0, 0.01, 0.1]))
    eps = float(rng.choice([1e-8, 1e-6]))
    max_norm = float(rng.choice([1e-3, 0.05, 1.0, 100.0]))
    defer = bool(rng.integers(0, 2))
    dtype = [torch.float32, torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 4))]
    dt = _NAMES[dtype]
    g_scale = 0.05 if dtype == torch.float16 else 1e-3  # fp16: keep (1 - beta2) g^2 above its subnormals
    if dtype == torch.float16:
        eps = float(rng.choice([1e-4, 1e-3]))  # 1e-8 rounds to 0 in fp16
    gen = torch.Generator(device=device).manual_seed(case)
    params = [torch.nn.Parameter((torch.randn(n, device=device, generator=gen) * 0.02).to(dtype)) for n in sizes]
    opt = ShardedOptimizer(params, OptimizerConfig(name="adamw", learning_rate=lr, betas=betas, weight_decay=wd,
                                                   eps=eps), norm_group=GroupHandle.trivial(), device=device,
                           defer_clip=defer)
    P = [_host_bits(p) for p in params]
    M = [np.zeros_like(a) for a in P]
    V = [np.zeros_like(a) for a in P]
    context = (f"case {case}: {len(sizes)} tensors, {dt} masters, lr {lr}, betas {betas}, wd {wd}, eps {eps}, "
               f"clip {max_norm}, defer {defer}")
    for step in (1, 2):
        for p in params:
            p.grad = (torch.randn(p.shape, device=device, generator=gen) * g_scale).to(dtype)
        G = [_host_bits(p.grad) for p in params]
        norm = float(opt.clip_grad_norm(max_norm))
        mul = oracle.clip_multiplier(norm, max_norm)
        opt.step()
        sc = oracle.adamw_scalars(lr=lr, beta1=betas[0], beta2=betas[1], eps=eps, weight_decay=wd, step=float(step))
        for p, a, g, m, v in zip(params, P, G, M, V):
            clipped = np.empty_like(g)
            oracle.adamw_step(a, g, m, v, sc, grad_mul=mul, dtype=dt, grad_out=clipped)
            assert np.array_equal(_host_bits(p.grad), g if defer else clipped), (context, step)
    for p, a, m, v in zip(params, P, M, V):
        state = opt.inner.state[p]
        assert np.array_equal(_host_bits(p), a), context
        assert np.array_equal(_host_bits(state["exp_avg"]), m), context
        assert np.array_equal(_host_bits(state["exp_avg_sq"]), v), context


@pytest.mark.parametrize("case", range(30))
def test_random_sgd_clip_steps(device, case):
    """Random SGD configurations (momentum, dampening, Nesterov, weight decay, learning
    rate), master dtypes (fp32, bf16, fp16), parameter lists and clip thresholds, three
    steps of ``clip_grad_norm`` + ``step`` (``optim/sharded_optimizer.py:121-126``, torch's
    ``_single_tensor_sgd``): parameters and momentum buffers bitwise the oracle's, and
    ``.grad`` the oracle's clipped gradient after an in-place clip."""
    from hybrid_training_amd import OptimizerConfig, ShardedOptimizer

    rng = np.random.default_rng(8000 + case)
    sizes = [int(rng.integers(1, 30000)) for _ in range(int(rng.integers(1, 25)))]
    lr = float(rng.choice([0.01, 0.05, 0.3]))
    momentum = float(rng.choice([0.0, 0.5, 0.9]))
    dampening = float(rng.choice([0.0, 0.25])) if momentum else 0.0
    nesterov = bool(rng.integers(0, 2)) and momentum > 0 and dampening == 0.0
    wd = float(rng.choice([0.0, 1e-4, 0.01]))
    max_norm = float(rng.choice([0.01, 1.0, 1e3]))
    defer = bool(rng.integers(0, 2))
    dtype = [torch.float32, torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 4))]
    dt = _NAMES[dtype]
    gen = torch.Generator(device=device).manual_seed(case)
    params = [torch.nn.Parameter(torch.randn(n, device=device, generator=gen).to(dtype)) for n in sizes]
    opt = ShardedOptimizer(params, OptimizerConfig(name="sgd", learning_rate=lr, momentum=momentum, weight_decay=wd),
                           norm_group=GroupHandle.trivial(), device=device, defer_clip=defer)
    for group in opt.inner.param_groups:
        group["dampening"] = dampening
        group["nesterov"] = nesterov
    P = [_host_bits(p) for p in params]
    B = [np.zeros_like(a) for a in P] if momentum else [None] * len(sizes)
    context = (f"case {case}: {len(sizes)} tensors, {dt} masters, lr {lr}, momentum {momentum}, "
               f"dampening {dampening}, nesterov {nesterov}, wd {wd}, clip {max_norm}, defer {defer}")
    for step in range(3):
        for p in params:
            p.grad = (torch.randn(p.shape, device=device, generator=gen) * 0.1).to(dtype)
        G = [_host_bits(p.grad) for p in params]
        mul = oracle.clip_multiplier(float(opt.clip_grad_norm(max_norm)), max_norm)
        opt.step()
        for p, a, g, b in zip(params, P, G, B):
            clipped = np.empty_like(g)
            oracle.sgd_step(a, g, b, lr=lr, momentum=momentum, dampening=dampening, weight_decay=wd,
                            nesterov=nesterov, first=step == 0, grad_mul=mul, dtype=dt, grad_out=clipped)
            assert np.array_equal(_host_bits(p.grad), g if defer else clipped), (context, step)
    for p, a, b in zip(params, P, B):
        assert np.array_equal(_host_bits(p), a), context
        if momentum:
            assert np.array_equal(_host_bits(opt.inner.state[p]["momentum_buffer"]), b), context


@pytest.mark.parametrize("case", range(30))
def test_random_loss_scaled_runs(device, case):
    """Six engine steps (``training/engine.py:392-400``: ``unscale_``, ``clip_grad_norm``,
    ``scaler.step``, ``update``) with random tensors, fp32 or bf16 gradients, deferred
    or eager multipliers, growth intervals and inf/nan injected on random steps
    (``optim/grad_scaler.py:164-269``).  A step is skipped exactly when some gradient is
    non-finite, leaving parameters and state untouched and halving the scale; clean
    steps are bitwise the oracle's AdamW with the unscale and the clip."""
    from hybrid_training_amd import GradScaler, GradScalerConfig, OptimizerConfig, ShardedOptimizer

    rng = np.random.default_rng(6000 + case)
    sizes = [int(rng.integers(1, 50000)) for _ in range(int(rng.integers(1, 6)))]
    bf16 = bool(rng.integers(0, 2))
    defer = bool(rng.integers(0, 2))
    interval = int(rng.integers(1, 4))
    max_norm = float(rng.choice([0.01, 1.0]))
    gen = torch.Generator(device=device).manual_seed(case)
    params = [torch.nn.Parameter(torch.randn(n, device=device, generator=gen) * 0.02) for n in sizes]
    for p in params:
        p.grad_dtype = None
    opt = ShardedOptimizer(params, OptimizerConfig(learning_rate=3e-4, betas=(0.9, 0.95), weight_decay=0.1),
                           norm_group=GroupHandle.trivial(), device=device, defer_clip=defer)
    scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=2.0**16, growth_interval=interval),
                        GroupHandle.trivial(), device, defer_unscale=defer)
    P = [p.detach().cpu().numpy().copy() for p in params]
    M = [np.zeros(n, np.float32) for n in sizes]
    V = [np.zeros(n, np.float32) for n in sizes]
    taken, tracker = 0, 0
    context = f"case {case}: sizes {sizes}, bf16 {bf16}, defer {defer}, interval {interval}, clip {max_norm}"
    for step in range(6):
        scale = scaler.scale_value
        grads = [torch.randn(n, device=device, generator=gen) * 1e-4 * scale for n in sizes]
        if bf16:
            grads = [g.to(torch.bfloat16) for g in grads]
        poison = rng.random() < 0.35
        if poison:
            victim = grads[int(rng.integers(0, len(grads)))]
            victim[int(rng.integers(0, victim.numel()))] = float(rng.choice([np.inf, -np.inf, np.nan]))
        for p, g in zip(params, grads):
            p.grad = g
        host = [(g.detach().cpu().view(torch.int16).numpy().view(np.uint16) if bf16 else g.detach().cpu().numpy())
                for g in grads]
        scaler.unscale_(params)
        norm = float(opt.clip_grad_norm(max_norm))
        stepped = scaler.step(opt, params, already_unscaled=True)
        scaler.update()
        # .grad as the reference leaves it (unscaled and clipped in place, the step taken
        # or skipped), or untouched with deferred multipliers
        mul = oracle.clip_multiplier(norm, max_norm)
        for p, g in zip(params, host):
            got = p.grad.detach().cpu()
            got = got.view(torch.int16).numpy().view(np.uint16) if bf16 else got.numpy()
            if defer:
                want = g
            else:
                want = np.empty_like(g)
                oracle.adamw_step(np.zeros(g.size, np.float32), g, np.zeros(g.size, np.float32),
                                  np.zeros(g.size, np.float32), (1.0,) * 7, unscale=1.0 / scale, grad_mul=mul,
                                  grad_out=want)
            dt = "bfloat16" if bf16 else "float32"
            nan = np.isnan(oracle.from_bits(want, dt))
            assert np.array_equal(np.isnan(oracle.from_bits(got, dt)), nan), (context, step)
            assert np.array_equal(got[~nan], want[~nan]), (context, step)
        opt.zero_grad(set_to_none=True)
        nonfinite = any(not torch.isfinite(g.float()).all() for g in grads)
        assert stepped == (not nonfinite), (context, step)
        if nonfinite:
            assert scaler.scale_value == max(scale / 2, 1.0) and scaler.state.growth_tracker == 0, (context, step)
            tracker = 0
        else:
            taken += 1
            sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=float(taken))
            for a, g, m, v in zip(P, host, M, V):
                oracle.adamw_step(a, g, m, v, sc, unscale=1.0 / scale, grad_mul=mul)
            tracker += 1
            grown = tracker == interval
            tracker = 0 if grown else tracker
            assert scaler.scale_value == (scale * 2 if grown else scale), (context, step)
        for p, a in zip(params, P):
            assert np.array_equal(p.detach().cpu().numpy().view(np.int32), a.view(np.int32)), (context, step)


@pytest.mark.parametrize("case", range(20))
def test_random_offloaded_runs(device, monkeypatch, case):
    """Optimizer-state offload (``optim/sharded_optimizer.py:284-296``, ``:342-353``) with
    random tensor sizes, chunk sizes (so chunks split tensors at random points and the
    two staging slots alternate), fp32, bf16 or fp16 masters, AdamW or SGD with momentum
    and deferred or eager clipping: three steps bitwise those of the in-HBM path, state
    and ``.grad`` included."""
    from hybrid_training_amd import OptimizerConfig, ShardedOptimizer
    from hybrid_training_amd.host_staging import HostStream

    rng = np.random.default_rng(4000 + case)
    monkeypatch.setattr(HostStream, "chunk_elems", int(rng.choice([1000, 4096, 65536])))
    sizes = [int(rng.integers(1, 40000)) for _ in range(int(rng.integers(1, 6)))]
    adamw = bool(rng.integers(0, 2))
    defer = bool(rng.integers(0, 2))
    dtype = [torch.float32, torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 4))]
    config = ({"name": "adamw", "learning_rate": 3e-4, "betas": (0.9, 0.95), "weight_decay": 0.1, "eps": 1e-4}
              if adamw else {"name": "sgd", "learning_rate": 0.05, "momentum": 0.9, "weight_decay": 0.01})
    gen = torch.Generator(device=device).manual_seed(case)
    init = [torch.randn(n, device=device, generator=gen).to(dtype) for n in sizes]
    runs = []
    for offload in (False, True):
        params = [torch.nn.Parameter(t.clone()) for t in init]
        opt = ShardedOptimizer(params, OptimizerConfig(**{**config, "cpu_offload_state": offload}),
                               norm_group=GroupHandle.trivial(), device=device, defer_clip=defer)
        runs.append((params, opt))
    context = f"case {case}: sizes {sizes}, {dtype} masters, adamw {adamw}, defer {defer}"
    for step in range(3):
        grads = [(torch.randn(n, device=device, generator=gen) * 0.1).to(dtype) for n in sizes]
        for params, opt in runs:
            for p, g in zip(params, grads):
                p.grad = g.clone()
            opt.clip_grad_norm(0.5)
            opt.step()
        for a, b in zip(runs[0][0], runs[1][0]):
            assert np.array_equal(_host_bits(a), _host_bits(b)), (context, step)
            assert np.array_equal(_host_bits(a.grad), _host_bits(b.grad)), (context, step)
    saved = [opt.state_dict()["state"] for _, opt in runs]
    for index, entry in saved[0].items():
        for key, value in entry.items():
            if torch.is_tensor(value):  # compare the bits at the tensor's own width
                other = saved[1][index][key]
                assert value.dtype == other.dtype, (context, index, key)
                assert value.dtype == (torch.float32 if key == "step" else dtype), (context, index, key)
                assert np.array_equal(_host_bits(value), _host_bits(other)), (context, index, key)


@pytest.mark.parametrize("case", range(30))
def test_random_weighted_norms(device, case):
    """The deterministic fp64 norm (``optim/sharded_optimizer.py:145-158``, ``:215-241``)
    over random segments of random fp32/bf16 tensors with the weights the path uses
    (the partitioned width, 0 over padding, 1/W for replicated parameters): the sum is
    within 1e-12 of a brute-force ``math.fsum`` of w * g^2 in fp64, the clip multiplier
    is the oracle's, and two runs agree bitwise."""
    import math

    from hybrid_training_amd.optim import gradient_norm_pass

    rng = np.random.default_rng(3000 + case)
    gen = torch.Generator(device=device).manual_seed(case)
    segments, terms = [], []
    for _ in range(int(rng.integers(1, 30))):
        dtype = [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
        n = int(rng.integers(1, 200_000))
        g = (torch.randn(n, device=device, generator=gen) * 1e-3).to(dtype)
        start = int(rng.integers(0, n))
        length = int(rng.integers(0, n - start + 1))
        weight = float(rng.choice([0.0, 0.125, 0.5, 1.0, 2.0, 8.0]))
        segments.append((g, start, length, weight))
        values = g[start:start + length].double().cpu().numpy()
        terms.extend((weight * values * values).tolist())
    max_norm = float(rng.choice([1e-3, 1.0, 1e6]))
    first = gradient_norm_pass(segments, device, max_norm=max_norm)
    second = gradient_norm_pass(segments, device, max_norm=max_norm)
    expect = math.fsum(terms)
    got = float(first.sum)
    assert abs(got - expect) <= 1e-12 * max(expect, 1e-300), (case, got, expect)
    assert float(first.sum) == float(second.sum) and float(first.norm) == float(second.norm)
    assert float(first.grad_mul) == oracle.clip_multiplier(float(first.norm), max_norm)


@pytest.mark.parametrize("case", range(12))
def test_random_checkpoint_save_and_load(device, tmp_path, case):
    """Random models saved by 1-5 FSDP writers after AdamW steps, through the on-disk
    format (``checkpoint/writer.py:433-567``, ``checkpoint/manifest.py:313-561``,
    ``checkpoint/reader.py:314-470``), and loaded at a random width: every reader's
    shard, ``exp_avg``, ``exp_avg_sq`` and ``step`` are the saved global values
    bitwise, and its padding stays zero."""
    from hybrid_training_amd import (OptimizerConfig, ShardedOptimizer, collect_flat_shard_payload,
                                     load_flat_shard_checkpoint, write_checkpoint)

    rng = np.random.default_rng(2000 + case)
    shapes = _shapes(rng)
    writers, readers = int(rng.integers(1, 6)), int(rng.integers(1, 7))
    steps = int(rng.integers(1, 3))
    total = sum(int(np.prod(s)) for s in shapes)
    gen = torch.Generator(device=device).manual_seed(case)

    def world(group, seed):
        init = torch.Generator(device=device).manual_seed(seed)
        named = [(f"p{i}", torch.nn.Parameter(torch.randn(s, device=device, generator=init)))
                 for i, s in enumerate(shapes)]
        handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(),
                                   MixedPrecisionConfig(), device, keep_originals=True) for r in range(group)]
        opts = [ShardedOptimizer([h.flat_param], OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                                 norm_group=GroupHandle.local_view("world", group, r), device=device)
                for r, h in enumerate(handles)]
        return handles, opts

    handles, opts = world(writers, 1)
    for _ in range(steps):
        for h, opt in zip(handles, opts):
            h.flat_param.grad = torch.randn(h.shard_numel, device=device, generator=gen) * 1e-2
            opt.step()
    payloads = [(r, *collect_flat_shard_payload(h, rank=r, optimizer=o)) for r, (h, o) in
                enumerate(zip(handles, opts))]
    path = write_checkpoint(tmp_path, steps, payloads, topology={"fsdp": writers})

    def flat_of(tensors):
        return torch.cat([t.detach().reshape(-1) for t in tensors])[:total]

    flat = flat_of([h.flat_param for h in handles])
    m = flat_of([o.inner.state[h.flat_param]["exp_avg"] for h, o in zip(handles, opts)])
    v = flat_of([o.inner.state[h.flat_param]["exp_avg_sq"] for h, o in zip(handles, opts)])
    new_handles, new_opts = world(readers, 99)   # different values: everything must come from disk
    context = f"case {case}: shapes {shapes}, {writers} -> {readers} ranks, {steps} steps"
    for r, (h, o) in enumerate(zip(new_handles, new_opts)):
        load_flat_shard_checkpoint(path, h, optimizer=o)
        start = r * h.shard_numel
        valid = max(0, min(h.shard_numel, total - start))
        state = o.inner.state[h.flat_param]
        assert torch.equal(h.flat_param.detach()[:valid], flat[start:start + valid]), (context, r)
        assert float(h.flat_param.detach()[valid:].abs().sum()) == 0.0, (context, r)
        assert torch.equal(state["exp_avg"][:valid], m[start:start + valid]), (context, r)
        assert torch.equal(state["exp_avg_sq"][:valid], v[start:start + valid]), (context, r)
        assert float(state["step"]) == float(steps), (context, r)


def _tiny_shapes(rng: np.random.Generator) -> list[tuple[int, ...]]:
    """One to three tensors of 0-5 elements: with up to 9 ranks most shards are padding."""
    shapes = [(int(rng.integers(0, 6)),) for _ in range(int(rng.integers(1, 4)))]
    if all(s[0] == 0 for s in shapes):
        shapes.append((1,))
    return shapes


@pytest.mark.parametrize("case", range(40))
def test_random_tiny_fsdp_configurations(device, monkeypatch, case):
    """The FSDP configurations above on models of a few elements, where most ranks own
    padding only: pack, gather, local share and ``no_sync`` bitwise the oracle's."""
    monkeypatch.setattr(sys.modules[__name__], "_shapes", _tiny_shapes)
    _fsdp_case(device, 5000 + case)


@pytest.mark.parametrize("case", range(20))
def test_random_tiny_checkpoint_save_and_load(device, tmp_path, monkeypatch, case):
    """The checkpoint round trips above on models of a few elements: writers and readers
    whose shards are all padding save nothing and load zero optimizer state."""
    monkeypatch.setattr(sys.modules[__name__], "_shapes", _tiny_shapes)
    test_random_checkpoint_save_and_load(device, tmp_path, 5000 + case)


@pytest.mark.parametrize("case", range(24))
def test_random_recorded_steps(device, case):
    """Random optimizer steps taken eagerly and by replaying a ``StepGraph`` recording of
    the same ``clip_grad_norm`` + ``step``: up to 40 tensors (launches split at 16, empty
    ones included), fp32 / bf16 / fp16 / float64 masters, AdamW (both lerp branches) or SGD
    (plain, momentum, Nesterov, weight decay), every clip placement, new gradients written
    into the recorded buffers before every step and the learning rate halved after the
    first replay.  Parameters, gradients, state, step counters and norms must be bitwise
    equal after every step."""
    from hybrid_training_amd import OptimizerConfig, ShardedOptimizer, StepGraph

    rng = np.random.default_rng(9000 + case)
    sizes = [int(rng.choice([0, 1, 7, 256, 1000, 4097])) if rng.random() < 0.3 else int(rng.integers(1, 20000))
             for _ in range(int(rng.integers(1, 41)))]
    dtype = [torch.float32, torch.float32, torch.bfloat16, torch.float16, torch.float64][int(rng.integers(0, 5))]
    name = ["adamw", "sgd"][int(rng.integers(0, 2))]
    placement = [{}, {"defer_clip": True}, {"clip_in_step": True}][int(rng.integers(0, 3))]
    lr = float(rng.choice([1e-4, 1e-3, 1e-2]))
    betas = [(0.9, 0.95), (0.8, 0.999), (0.4, 0.9)][int(rng.integers(0, 3))]
    wd = float(rng.choice([0.0, 0.01]))
    momentum = float(rng.choice([0.0, 0.9]))
    nesterov = momentum != 0 and bool(rng.integers(0, 2))
    eps = float(rng.choice([1e-4, 1e-3])) if dtype == torch.float16 else 1e-8
    g_scale = 0.05 if dtype == torch.float16 else 1e-3
    max_norm = float(rng.choice([1e-3, 0.05, 1.0, 100.0]))
    config = OptimizerConfig(name=name, learning_rate=lr, betas=betas, weight_decay=wd, eps=eps, momentum=momentum)
    context = (f"case {case}: {len(sizes)} tensors, {_NAMES[dtype]}, {name}, {placement}, lr {lr}, betas {betas}, "
               f"wd {wd}, momentum {momentum}, nesterov {nesterov}, clip {max_norm}")

    def build():
        gen = torch.Generator(device=device).manual_seed(case)
        params = [torch.nn.Parameter((torch.randn(n, device=device, generator=gen) * 0.02).to(dtype)) for n in sizes]
        opt = ShardedOptimizer(params, config, norm_group=GroupHandle.trivial(), device=device, **placement)
        if nesterov:
            for group in opt.inner.param_groups:
                group["nesterov"] = True
        for p in params:
            p.grad = torch.zeros_like(p)  # the gradient buffers every step writes into
        return params, opt

    def fill(params, k):
        gen = torch.Generator(device=device).manual_seed(1000 * case + k)
        for p in params:
            p.grad.copy_((torch.randn(p.shape, device=device, generator=gen) * g_scale).to(dtype))

    (pa, oa), (pb, ob) = build(), build()
    for params, opt in ((pa, oa), (pb, ob)):
        fill(params, 0)
        opt.clip_grad_norm(max_norm)
        opt.step()
    graph = StepGraph(lambda: (ob.clip_grad_norm(max_norm), ob.step())[0])
    for k in range(1, 4):
        if k == 2:
            oa.set_learning_rate(lr / 2)
            ob.set_learning_rate(lr / 2)
        fill(pa, k)
        fill(pb, k)
        norm = oa.clip_grad_norm(max_norm)
        oa.step()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(norm, graph.output), (context, k)
        for a, b in zip(pa, pb):
            assert torch.equal(a, b) and torch.equal(a.grad, b.grad), (context, k)
            sa, sb = oa.inner.state[a], ob.inner.state[b]
            assert sa.keys() == sb.keys(), context
            for key in sa:
                assert torch.equal(sa[key], sb[key]), (context, k, key)


@pytest.mark.parametrize("case", range(16))
def test_random_recorded_ddp_steps(device, case):
    """Random data-parallel tails taken eagerly and by replaying a ``StepGraph``
    recording: parameters of random shapes in gradient buckets of a random cap (the
    gradients bound as bucket views after the first step, so each pack divides them in
    place by the group size), group sizes 1 to 8, fp32 / bf16 / float64 parameters, AdamW
    or SGD with every clip placement.  Buckets, parameters, state and norms must be
    bitwise equal after every step."""
    from hybrid_training_amd import BucketedGradients, DDPConfig, OptimizerConfig, ShardedOptimizer, StepGraph

    rng = np.random.default_rng(9500 + case)
    shapes = [tuple(int(d) for d in rng.integers(1, 40, int(rng.integers(1, 3)))) for _ in range(int(rng.integers(1, 13)))]
    dtype = [torch.float32, torch.bfloat16, torch.float64][int(rng.integers(0, 3))]
    world = int(rng.integers(1, 9))
    cap_mb = float(rng.choice([0.5, 2.0, 8.0])) / 1024
    name = ["adamw", "sgd"][int(rng.integers(0, 2))]
    placement = [{}, {"defer_clip": True}, {"clip_in_step": True}][int(rng.integers(0, 3))]
    max_norm = float(rng.choice([0.01, 1.0, 100.0]))
    config = OptimizerConfig(name=name, learning_rate=1e-3, weight_decay=0.01, momentum=0.9)
    context = f"case {case}: shapes {shapes}, {_NAMES[dtype]}, W={world}, cap {cap_mb} MiB, {name}, {placement}"

    def build():
        gen = torch.Generator(device=device).manual_seed(case)
        named = [(f"p{i}", torch.nn.Parameter((torch.randn(s, device=device, generator=gen) * 0.02).to(dtype)))
                 for i, s in enumerate(shapes)]
        group = GroupHandle.local_view("data_parallel", world, 0) if world > 1 else GroupHandle.trivial()
        ddp = BucketedGradients(named, group, DDPConfig(bucket_cap_mb=cap_mb))
        params = [p for _, p in named]
        opt = ShardedOptimizer(params, config, norm_group=GroupHandle.trivial(), device=device, **placement)
        return params, ddp, opt

    def fill(params, k):
        gen = torch.Generator(device=device).manual_seed(1000 * case + k)
        for p in params:
            g = (torch.randn(p.shape, device=device, generator=gen) * 1e-2).to(dtype)
            if p.grad is None:
                p.grad = g
            else:
                p.grad.copy_(g)

    def step(params, ddp, opt):
        ddp.synchronize()
        norm = opt.clip_grad_norm(max_norm)
        opt.step()
        return norm

    a, b = build(), build()
    for params, ddp, opt in (a, b):
        fill(params, 0)
        step(params, ddp, opt)
    graph = StepGraph(lambda: step(*b))
    for k in range(1, 4):
        fill(a[0], k)
        fill(b[0], k)
        norm = step(*a)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(norm, graph.output), (context, k)
        for ba, bb in zip(a[1]._buckets, b[1]._buckets):
            assert torch.equal(ba.buffer, bb.buffer), (context, k, "bucket")
        for pa, pb in zip(a[0], b[0]):
            assert torch.equal(pa, pb), (context, k)
            sa, sb = a[2].inner.state[pa], b[2].inner.state[pb]
            assert sa.keys() == sb.keys(), context
            for key in sa:
                assert torch.equal(sa[key], sb[key]), (context, k, key)
