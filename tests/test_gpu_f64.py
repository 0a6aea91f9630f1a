"""GPU parity of the float64 path: parameters, gradients and state in float64.

With mixed precision off the reference's flat shards, gradients and optimizer state
have the parameters' dtype (``parallel/fsdp.py:379-393``), float64 included
(``config.py:55-56``), and torch's AdamW / SGD step them in double
(``optim/sharded_optimizer.py:111-126``).  Checked here against the oracle, itself pinned
bitwise to torch's float64 CPU optimizers (``tests/test_oracle_f64.py``):

* ``hbt_adamw_step_f64`` / ``hbt_sgd_step_f64`` bitwise the oracle over tails, a misaligned
  tensor, both lerp branches, the unscale and clip multiplies and the gradient write-back;
* ``ShardedOptimizer`` on float64 parameters: 10 clipped AdamW steps bitwise the oracle and
  within 1e-15 of torch's CPU AdamW (whose float64 sqrt is not correctly rounded), SGD
  bitwise torch; ``.grad`` clipped in place bitwise torch's ``grad.mul_(coefficient)``;
* the float64 norm within 1e-13 of the correctly rounded sum of squares;
* an FSDP unit of float64 parameters with mixed precision off: pack, AVG local share in
  float64 (G = 3 divides, G = 4 and 8 multiply by the exact reciprocal) and its norm
  partials, then the clipped step, bitwise the oracle;
* a float64 DDP bucket's AVG divide bitwise numpy's double division, IEEE specials included;
* the loss scaler on float64 gradients: the unscale in double, skip on overflow;
* the vectorised conversions through double (every pair with float64, and bf16 <-> fp16)
  on aligned plans bitwise torch's ``Tensor.to``, NaNs as NaNs; the float64 divide on
  aligned and misaligned plans bitwise numpy.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import (
    BucketedGradients,
    DDPConfig,
    FlatParamHandle,
    FSDPConfig,
    GradScaler,
    GradScalerConfig,
    GroupHandle,
    MixedPrecisionConfig,
    OptimizerConfig,
    ShardedOptimizer,
    _native,
)
from hybrid_training_amd.optim import gradient_norm_pass

pytestmark = pytest.mark.gpu


def _u64(t) -> np.ndarray:
    a = t.detach().cpu().numpy() if torch.is_tensor(t) else np.asarray(t)
    return np.ascontiguousarray(a, dtype=np.float64).view(np.uint64)


def _host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().astype(np.float64).copy()


def _launch_adamw64(ps, gs, ms, vs, scalars, *, unscale=1.0, grad_mul=None, flags=0):
    lib = _native.library()
    status = lib.hbt_adamw_step_f64(
        _native.pointer_array([t.data_ptr() for t in ps]), _native.pointer_array([t.data_ptr() for t in gs]),
        _native.pointer_array([t.data_ptr() for t in ms]), _native.pointer_array([t.data_ptr() for t in vs]),
        _native.int64_array([t.numel() for t in ps]), len(ps), unscale,
        None if grad_mul is None else grad_mul.data_ptr(), *scalars, flags,
        ctypes.c_void_p(_native.stream_of(ps[0].device)))
    _native.check(status, "test.hbt_adamw_step_f64")


@pytest.mark.parametrize("betas", [(0.9, 0.95), (0.3, 0.9)])
@pytest.mark.parametrize("write_back", [False, True])
def test_adamw_f64_kernel_bitwise_vs_oracle(device, betas, write_back):
    sizes = [1, 63, 64, 65, 127, 128, 129, 4099, 100_003]
    gen = torch.Generator(device=device).manual_seed(5)
    base = torch.randn(sum(sizes) + 1, device=device, generator=gen, dtype=torch.float64) * 0.02
    ps, cursor = [], 1  # the first tensor starts one element in: the scalar path
    for n in sizes:
        ps.append(base[cursor:cursor + n])
        cursor += n
    gs = [torch.randn(n, device=device, generator=gen, dtype=torch.float64) * 1e-2 for n in sizes]
    ms = [torch.randn(n, device=device, generator=gen, dtype=torch.float64) * 1e-3 for n in sizes]
    vs = [torch.rand(n, device=device, generator=gen, dtype=torch.float64) * 1e-5 for n in sizes]
    host = [(_host(p), _host(g), _host(m), _host(v)) for p, g, m, v in zip(ps, gs, ms, vs)]
    mul = 0.37191827364912  # not a power of two, not an fp32 value
    unscale = 1.0 / 1000.0
    scalars = oracle.adamw_scalars(lr=3e-4, beta1=betas[0], beta2=betas[1], eps=1e-8, weight_decay=0.1, step=3.0)
    _launch_adamw64(ps, gs, ms, vs, scalars, unscale=unscale,
                    grad_mul=torch.tensor([mul], dtype=torch.float64, device=device),
                    flags=_native.STEP_WRITE_GRAD if write_back else 0)
    for (P, G, M, V), p, g, m, v in zip(host, ps, gs, ms, vs):
        out = np.empty_like(G)
        oracle.adamw_step_f64(P, G, M, V, scalars, unscale=unscale, grad_mul=mul, grad_out=out)
        assert np.array_equal(_u64(p), P.view(np.uint64)), p.numel()
        assert np.array_equal(_u64(m), M.view(np.uint64)), p.numel()
        assert np.array_equal(_u64(v), V.view(np.uint64)), p.numel()
        assert np.array_equal(_u64(g), (out if write_back else G).view(np.uint64)), p.numel()


def test_sharded_adamw_f64_matches_torch_and_the_oracle(device):
    """Ten clipped steps on three float64 tensors (one misaligned view): parameters and
    state bitwise the oracle, within 1e-15 of torch's CPU AdamW; ``.grad`` clipped in place
    before the step as torch's ``grad.mul_(coefficient)`` leaves it."""
    sizes = (70_001, 4096, 33)
    gen = torch.Generator().manual_seed(21)
    p0 = [torch.randn(n, generator=gen, dtype=torch.float64) * 0.02 for n in sizes]
    storage = torch.zeros(sum(sizes) + 1, dtype=torch.float64, device=device)
    params, cursor = [], 1
    for t in p0:
        view = storage[cursor:cursor + t.numel()]
        view.copy_(t.to(device))
        params.append(torch.nn.Parameter(view))
        cursor += t.numel()
    config = OptimizerConfig(learning_rate=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    opt = ShardedOptimizer(params, config, norm_group=GroupHandle.trivial(), device=device)
    ref = [torch.nn.Parameter(t.clone()) for t in p0]
    ref_opt = torch.optim.AdamW(ref, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=False)
    host = [t.numpy().copy() for t in p0]
    M = [np.zeros(n) for n in sizes]
    V = [np.zeros(n) for n in sizes]
    worst = 0.0
    for step in range(1, 11):
        grads = [torch.randn(n, generator=gen, dtype=torch.float64) * 1e-2 for n in sizes]
        for p, g in zip(params, grads):
            p.grad = g.to(device)
        norm = float(opt.clip_grad_norm(1.0))
        exact = math.sqrt(math.fsum(float(x) * float(x) for g in grads for x in g.numpy()))
        assert abs(norm - exact) <= 1e-14 * exact
        coef = 1.0 / (norm + 1e-6)
        assert coef < 1.0
        for p, g in zip(params, grads):  # clipped in place before the step, as the reference
            assert torch.equal(p.grad.cpu(), g.clone().mul_(coef))
        opt.step()
        for r, g in zip(ref, grads):
            r.grad = g.clone().mul_(coef)
        ref_opt.step()
        sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=float(step))
        for k, g in enumerate(grads):
            oracle.adamw_step_f64(host[k], g.numpy(), M[k], V[k], sc, grad_mul=oracle.clip_multiplier64(norm, 1.0))
            assert np.array_equal(_u64(params[k]), host[k].view(np.uint64)), (step, k)
            state = opt.inner.state[params[k]]
            assert np.array_equal(_u64(state["exp_avg"]), M[k].view(np.uint64))
            assert np.array_equal(_u64(state["exp_avg_sq"]), V[k].view(np.uint64))
            want = ref[k].detach().numpy()
            worst = max(worst, float(np.max(np.abs(host[k] - want) / np.maximum(np.abs(want), 3e-4))))
    assert worst <= 1e-15, worst


@pytest.mark.parametrize("momentum,nesterov,wd", [(0.0, False, 0.0), (0.9, False, 0.01), (0.9, True, 0.0)])
def test_sharded_sgd_f64_matches_torch(device, momentum, nesterov, wd):
    """SGD on float64 parameters, clipped in place: bitwise torch's CPU SGD over three
    steps (no square root on this path, so no tolerance)."""
    sizes = (10_007, 129, 1)
    gen = torch.Generator().manual_seed(8)
    p0 = [torch.randn(n, generator=gen, dtype=torch.float64) for n in sizes]
    params = [torch.nn.Parameter(t.to(device)) for t in p0]
    opt = ShardedOptimizer(params, OptimizerConfig(name="sgd", learning_rate=0.05, momentum=momentum,
                                                   weight_decay=wd),
                           norm_group=GroupHandle.trivial(), device=device)
    for group in opt.inner.param_groups:
        group["nesterov"] = nesterov
    ref = [torch.nn.Parameter(t.clone()) for t in p0]
    ref_opt = torch.optim.SGD(ref, lr=0.05, momentum=momentum, weight_decay=wd, nesterov=nesterov, foreach=False)
    for step in range(3):
        grads = [torch.randn(n, generator=gen, dtype=torch.float64) for n in sizes]
        for p, g in zip(params, grads):
            p.grad = g.to(device)
        norm = float(opt.clip_grad_norm(1.0))
        opt.step()
        for r, g in zip(ref, grads):
            r.grad = g.clone().mul_(1.0 / (norm + 1e-6))
        ref_opt.step()
        for p, r in zip(params, ref):
            assert np.array_equal(_u64(p), _u64(r)), step
            if momentum:
                assert np.array_equal(_u64(opt.inner.state[p]["momentum_buffer"]),
                                      _u64(ref_opt.state[r]["momentum_buffer"])), step


def test_f64_norm_pass_is_reproducible_and_weighted(device):
    gen = torch.Generator(device=device).manual_seed(3)
    grads = [torch.randn(n, device=device, generator=gen, dtype=torch.float64) for n in (1, 16383, 16384, 16385,
                                                                                          200_003)]
    segments = [(g, 0, g.numel(), 1.0) for g in grads] + [(grads[-1], 5, 1000, 0.25)]
    first = gradient_norm_pass(segments, device, max_norm=0.0)
    again = gradient_norm_pass(segments, device, max_norm=0.0)
    exact = math.fsum([float(x) * float(x) for g in grads for x in g.cpu().numpy()]
                      + [0.25 * float(x) * float(x) for x in grads[-1].cpu().numpy()[5:1005]])
    assert abs(float(first.sum) - exact) <= 1e-13 * exact
    assert float(first.sum) == float(again.sum)
    assert abs(oracle.sqnorm_f64(grads[-1].cpu().numpy()) - float(gradient_norm_pass(
        [(grads[-1], 0, grads[-1].numel(), 1.0)], device, max_norm=0.0).sum)) <= 1e-13 * exact


@pytest.mark.parametrize("group", [3, 4, 8])
def test_f64_fsdp_unit_without_mixed_precision(device, group):
    """float64 parameters, mixed precision off: the shard packs bitwise, the gradient shard
    is the oracle's float64 AVG local share (padding zero), the clip takes its norm from
    the share's partials, and the clipped AdamW step is bitwise the oracle's."""
    shapes = [(25, 14), (25,), (25, 25), (25,), (7, 25), (7,)]
    gen = torch.Generator(device=device).manual_seed(4)
    originals = [torch.randn(s, device=device, generator=gen, dtype=torch.float64) * 0.1 for s in shapes]
    total = sum(t.numel() for t in originals)
    handles = []
    for rank in range(group):
        named = [(f"p{i}", torch.nn.Parameter(t.clone())) for i, t in enumerate(originals)]
        handles.append(FlatParamHandle(named, None, GroupHandle.local_view("shard", group, rank), FSDPConfig(),
                                       MixedPrecisionConfig(enabled=False), device))
    shard = handles[0].shard_numel
    flat = torch.cat([t.reshape(-1) for t in originals]).cpu()
    full_grads = [torch.randn(shard * group, device=device, generator=gen, dtype=torch.float64) * 1e-2
                  for _ in range(group)]
    for g in full_grads:
        g[total:] = 0.0
    host_grads = [g.cpu().numpy() for g in full_grads]
    for rank, handle in enumerate(handles):
        assert handle.flat_param.dtype == torch.float64
        want = torch.zeros(shard, dtype=torch.float64)
        lo, hi = rank * shard, min(total, (rank + 1) * shard)
        if hi > lo:
            want[: hi - lo] = flat[lo:hi]
        assert torch.equal(handle.flat_param.detach().cpu(), want)
        out = handle.reduce_scatter_gradient(full_grads[rank], peer_grads=full_grads)
        valid = max(0, min(shard, total - rank * shard))
        expect = oracle.local_share(host_grads, rank, shard, valid, float(group), "float64", out="float64")
        assert out.dtype == torch.float64 and np.array_equal(_u64(out), expect.view(np.uint64)), rank
        param = handle.flat_param
        param.grad = out
        opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=1e-3, betas=(0.9, 0.999), weight_decay=0.01),
                               norm_group=GroupHandle.local_view("world", group, rank), device=device)
        P = _host(param)
        norm = float(opt.clip_grad_norm(1e-3))  # from the share's partials; clips
        exact = math.sqrt(math.fsum(float(x) * float(x) for x in expect))
        assert abs(norm - exact) <= 1e-13 * max(exact, 1e-300)
        opt.step()
        sc = oracle.adamw_scalars(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, step=1.0)
        oracle.adamw_step_f64(P, expect, np.zeros(shard), np.zeros(shard), sc,
                              grad_mul=oracle.clip_multiplier64(norm, 1e-3))
        assert np.array_equal(_u64(param), P.view(np.uint64)), rank


def test_f64_master_over_a_float32_reduce(device):
    """Mixed precision with a float64 master and a float32 reduce dtype: the share is
    reduced in float32, then widened exactly."""
    named = [("w", torch.nn.Parameter(torch.randn(1000, device=device)))]
    mp = MixedPrecisionConfig(enabled=True, param_dtype="float32", reduce_dtype="float32", master_dtype="float64")
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", 3, r), FSDPConfig(), mp, device,
                               keep_originals=True) for r in range(3)]
    shard = handles[0].shard_numel
    grads = [torch.randn(shard * 3, device=device) for _ in range(3)]
    for g in grads:
        g[1000:] = 0.0
    host = [g.cpu().numpy() for g in grads]
    for rank, h in enumerate(handles):
        out = h.reduce_scatter_gradient(grads[rank], peer_grads=grads)
        valid = max(0, min(shard, 1000 - rank * shard))
        expect = oracle.local_share(host, rank, shard, valid, 3.0, "float32").astype(np.float64)
        assert out.dtype == torch.float64 and np.array_equal(_u64(out), expect.view(np.uint64))


@pytest.mark.parametrize("world", [3, 8])
def test_f64_bucket_pack_divides_in_double(device, world):
    shapes = [(4099,), (33, 17), (1,)]
    named = [(f"w{i}", torch.nn.Parameter(torch.empty(s, device=device, dtype=torch.float64)))
             for i, s in enumerate(shapes)]
    gen = torch.Generator(device=device).manual_seed(19)
    for _, p in named:
        g = torch.randn(p.numel(), device=device, generator=gen, dtype=torch.float64)
        specials = [float("inf"), -float("inf"), float("nan"), -0.0, torch.finfo(torch.float64).max, 5e-324, 3e-310]
        k = min(len(specials), g.numel())
        g[:k] = torch.tensor(specials[:k], dtype=torch.float64, device=device)
        p.grad = g.reshape(p.shape)
    expect = {name: p.grad.detach().cpu().numpy().reshape(-1) / np.float64(world) for name, p in named}
    ddp = BucketedGradients(named, GroupHandle.local_view("data_parallel", world, 0), DDPConfig())
    ddp.synchronize()
    for name, p in named:
        got = p.grad.detach().cpu().numpy().reshape(-1)
        nan = np.isnan(expect[name])
        assert np.array_equal(np.isnan(got), nan), name
        assert np.array_equal(got[~nan].view(np.uint64), expect[name][~nan].view(np.uint64)), name


def test_f64_divide_on_misaligned_plans(device):
    """The float64 AVG divide over records at odd element offsets (the element-wise kernel)
    and aligned ones (the vector kernel), by 3 and by 4."""
    src = torch.randn(10_000, device=device, dtype=torch.float64)
    for divisor in (3.0, 4.0):
        for offset in (0, 1):
            dst = torch.zeros(10_000, device=device, dtype=torch.float64)
            plan = _native.CopyPlan(device)
            plan.add(src, offset, dst, offset, 9_000 + offset)
            plan.run(src_dtype=torch.float64, dst_dtype=torch.float64, op=_native.COPY_OP_DIVIDE, divisor=divisor)
            want = src.cpu().numpy()[offset:9_000 + 2 * offset] / divisor
            got = dst.cpu().numpy()[offset:9_000 + 2 * offset]
            assert np.array_equal(got.view(np.uint64), want.view(np.uint64)), (divisor, offset)
            assert not dst[:offset].any() and not dst[9_000 + 2 * offset:].any()


_PAIRS = [(a, b) for a in (torch.float64, torch.float32, torch.bfloat16, torch.float16)
          for b in (torch.float64, torch.float32, torch.bfloat16, torch.float16)
          if a != b and (torch.float64 in (a, b) or {a, b} == {torch.bfloat16, torch.float16})]


@pytest.mark.parametrize("src_dtype, dst_dtype", _PAIRS)
def test_aligned_conversions_through_double(device, src_dtype, dst_dtype):
    """The vector kernel of the conversions through double (aligned records: every
    destination and source on a 16-byte boundary), tails of every length and several
    chunks per record, with IEEE specials: bitwise torch's CPU ``Tensor.to``, NaN as NaN."""
    gen = torch.Generator().manual_seed(6)
    sizes = [1, 5, 127, 128, 129, 511, 512, 513, 4099, 100_003]
    values = []
    for n in sizes:
        exps = torch.rand(n, generator=gen, dtype=torch.float64) * 80 - 40
        v = torch.randn(n, generator=gen, dtype=torch.float64) * torch.pow(2.0, exps)
        specials = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 65504.0, 65520.0, 1e-8,
                                 3.5e38, 1e-40, 1e-300, 1.0 + 2.0**-30], dtype=torch.float64)
        k = min(n, specials.numel())
        v[:k] = specials[:k]
        values.append(v.to(src_dtype))
    srcs = [v.to(device) for v in values]
    dsts = [torch.empty(v.numel(), dtype=dst_dtype, device=device) for v in values]
    plan = _native.CopyPlan(device)
    for s, d in zip(srcs, dsts):
        plan.add(s, 0, d, 0, s.numel())
    plan.run(src_dtype=src_dtype, dst_dtype=dst_dtype)
    for v, d in zip(values, dsts):
        want = v.to(dst_dtype)
        got = d.cpu()
        nan = torch.isnan(want)
        assert torch.equal(torch.isnan(got), nan)
        ints = {8: torch.int64, 4: torch.int32, 2: torch.int16}[want.element_size()]
        assert torch.equal(got[~nan].view(ints) if got.dim() else got, want[~nan].view(ints)), v.numel()


def test_scale_inplace_f64_multiplies_in_double(device):
    lib = _native.library()
    x = torch.randn(100_003, device=device, dtype=torch.float64)
    x[7] = float("nan")
    before = x.cpu().numpy().copy()
    mul = torch.tensor([0.7123456789012345], dtype=torch.float64, device=device)
    status = lib.hbt_scale_inplace_f64(_native.pointer_array([x.data_ptr()]), _native.int64_array([x.numel()]), 1,
                                       1.0 / 3.0, mul.data_ptr(), ctypes.c_void_p(_native.stream_of(device)))
    _native.check(status, "test.hbt_scale_inplace_f64")
    want = (before * (1.0 / 3.0)) * 0.7123456789012345
    got = x.cpu().numpy()
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint64), want[ok].view(np.uint64)) and np.isnan(got[7])
    # both factors 1: nothing is read or written, a NaN payload included
    y = torch.randn(1000, device=device, dtype=torch.float64)
    y.view(torch.int64)[3] = 0x7FF0000000000123
    bits = y.view(torch.int64).cpu().clone()
    one = torch.ones(1, dtype=torch.float64, device=device)
    _native.check(lib.hbt_scale_inplace_f64(_native.pointer_array([y.data_ptr()]), _native.int64_array([1000]), 1,
                                            1.0, one.data_ptr(), ctypes.c_void_p(_native.stream_of(device))), "test")
    assert torch.equal(y.view(torch.int64).cpu(), bits)


@pytest.mark.parametrize("defer", [False, True])
def test_loss_scaler_on_f64_gradients(device, defer):
    """A float64 gradient is unscaled in double (``grad.mul_(1/scale)`` with the Python
    double), at once even with ``defer_unscale``; an inf skips the step and backs off."""
    param = torch.nn.Parameter(torch.randn(5000, device=device, dtype=torch.float64) * 0.02)
    opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=1e-3), norm_group=GroupHandle.trivial(),
                           device=device)
    scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=1000.0), GroupHandle.trivial(), device,
                        defer_unscale=defer)
    g = torch.randn(5000, dtype=torch.float64) * 1000.0
    param.grad = g.to(device)
    assert not scaler.unscale_([param])
    assert torch.equal(param.grad.cpu(), g.clone().mul_(1.0 / 1000.0))
    before = param.detach().clone()
    assert scaler.step(opt, [param], already_unscaled=True)
    assert not torch.equal(param.detach(), before)
    scaler.update()
    bad = g.clone()
    bad[10] = float("inf")
    param.grad = bad.to(device)
    before = param.detach().clone()
    assert scaler.unscale_([param])
    assert not scaler.step(opt, [param], already_unscaled=True)
    assert torch.equal(param.detach(), before)
    scaler.update()
    assert scaler.state.scale == 500.0
