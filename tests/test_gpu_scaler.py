"""GPU parity of the loss-scaled, clipped AdamW step (the mixed-precision shard path).

Reference semantics (``optim/grad_scaler.py:164-269``, ``training/engine.py:392-400``):
unscale, check for non-finite values, clip, skip the step on overflow and back the
scale off, otherwise step.  bf16 gradients are read as exactly widened fp32 master
gradients.  Checked against the oracle bitwise (update) and to 1e-12 (norm), at
reduced size, and at the full size of one Llama-3-70B FSDP rank at W=8
(8,819,213,312 parameters, ~123 GB resident) on a random subset of elements.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import GradScaler, GradScalerConfig, GroupHandle, OptimizerConfig, ShardedOptimizer
from hybrid_training_amd.errors import ShardingError, UnsupportedFeatureError

pytestmark = pytest.mark.gpu

SCALE = 65536.0


def _setup(param, defer=True):
    # bf16 gradients on fp32 master parameters: torch requires the grad dtype to be declared.
    param.grad_dtype = None
    opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=3e-4, betas=(0.9, 0.95), weight_decay=0.1),
                           norm_group=GroupHandle.trivial(), device=param.device, defer_clip=defer)
    scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=SCALE), GroupHandle.trivial(), param.device,
                        defer_unscale=defer)
    return opt, scaler


def _engine_step(opt, scaler, param, max_norm=1.0):
    """training/engine.py:392-400: unscale_, clip_grad_norm, scaler.step, update, zero_grad."""
    scaler.unscale_([param])
    norm = opt.clip_grad_norm(max_norm)
    stepped = scaler.step(opt, [param], already_unscaled=True)
    scaler.update()
    opt.zero_grad(set_to_none=True)
    return norm, stepped


def _bf16_bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def test_overflow_skip_then_clean_step(device, caplog):
    n = 1 << 22
    gen = torch.Generator(device=device).manual_seed(5)
    param = torch.nn.Parameter(torch.randn(n, device=device, generator=gen) * 0.02)
    p0 = param.detach().clone()
    opt, scaler = _setup(param)
    g = (torch.randn(n, device=device, generator=gen) * 1e-4 * SCALE).to(torch.bfloat16)
    bad = torch.randint(0, n, (n // 1000,), device=device, generator=gen)
    g[bad[: bad.numel() // 2]] = float("inf")
    g[bad[bad.numel() // 2 :]] = float("nan")
    param.grad = g
    with caplog.at_level("WARNING"):
        norm, stepped = _engine_step(opt, scaler, param)
    assert not stepped and not torch.isfinite(norm)
    assert "skipping optimizer step 1" in caplog.text  # logged as the reference does
    assert torch.equal(param.detach(), p0)
    assert scaler.scale_value == SCALE / 2 and scaler.state.skipped_steps == 1
    assert opt.inner.state[param] == {} or float(opt.inner.state[param]["step"]) == 0.0

    scale = scaler.scale_value
    g = (torch.randn(n, device=device, generator=gen) * 1e-4 * scale).to(torch.bfloat16)
    G = _bf16_bits(g)
    param.grad = g
    norm, stepped = _engine_step(opt, scaler, param)
    assert stepped and scaler.state.total_steps == 2 and scaler.state.growth_tracker == 1
    ref = oracle.sqnorm(G, unscale=1.0 / scale)
    assert abs(float(norm) ** 2 - ref) <= 1e-12 * ref
    P = p0.cpu().numpy()
    M = np.zeros(n, np.float32)
    V = np.zeros(n, np.float32)
    sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=1.0)
    oracle.adamw_step(P, G, M, V, sc, unscale=1.0 / scale, grad_mul=oracle.clip_multiplier(float(norm), 1.0))
    assert np.array_equal(param.detach().cpu().numpy().view(np.int32), P.view(np.int32))


def test_eager_and_deferred_unscale_agree_for_fp32_grads(device):
    n = 300_001
    g = torch.randn(n, device=device) * 1e-3 * SCALE
    p0 = torch.randn(n, device=device) * 0.02
    results = []
    for defer in (False, True):
        param = torch.nn.Parameter(p0.clone())
        opt, scaler = _setup(param, defer=defer)
        param.grad = g.clone()
        norm, stepped = _engine_step(opt, scaler, param, max_norm=0.5)
        assert stepped
        results.append((param.detach().clone(), float(norm)))
    assert torch.equal(results[0][0], results[1][0]) and results[0][1] == results[1][1]


def test_unscale_return_value_is_the_overflow_flag(device):
    param = torch.nn.Parameter(torch.zeros(10, device=device))
    for defer in (False, True):
        opt, scaler = _setup(param, defer=defer)
        param.grad = torch.ones(10, device=device)
        assert not bool(scaler.unscale_([param]))
        param.grad = torch.ones(10, device=device)
        param.grad[3] = float("nan")
        assert bool(scaler.unscale_([param]))


def test_unscale_refuses_gradients_the_kernel_cannot_address(device):
    """The in-place scale reads ``numel`` consecutive elements from a gradient's address:
    a strided gradient is refused (``ShardingError``) rather than scaled in the wrong
    places, and a float64 one is unscaled in double."""
    scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=1024.0), GroupHandle.trivial(), device)
    p = torch.nn.Parameter(torch.zeros(10, device=device))
    storage = torch.arange(20.0, device=device)
    p.grad = storage[::2]
    with pytest.raises(ShardingError, match="must be dense"):
        scaler.unscale_([p])
    assert torch.equal(storage, torch.arange(20.0, device=device))  # nothing was touched
    q = torch.nn.Parameter(torch.zeros(10, device=device, dtype=torch.float64))
    q.grad = torch.ones(10, device=device, dtype=torch.float64)
    assert not scaler.unscale_([q])
    assert torch.equal(q.grad, torch.full((10,), 1.0 / 1024.0, dtype=torch.float64, device=device))


def test_llama3_70b_rank_shard_full_size(device):
    n = 8_819_213_312
    gen = torch.Generator(device=device).manual_seed(70)
    param = torch.nn.Parameter(torch.empty(n, device=device))
    grad = torch.empty(n, dtype=torch.bfloat16, device=device)
    chunk = 1 << 30
    for start in range(0, n, chunk):
        stop = min(n, start + chunk)
        param.data[start:stop].normal_(0.0, 0.02, generator=gen)
        grad[start:stop] = (torch.randn(stop - start, device=device, generator=gen) * (1e-4 * SCALE)).to(torch.bfloat16)
    idx = torch.randint(0, n, (1 << 20,), device=device, generator=gen)
    idx[0], idx[1] = 0, n - 1
    P = param.detach()[idx].cpu().numpy()
    opt, scaler = _setup(param)
    # 0.1 % non-finite: the step is skipped.
    bad = torch.randint(0, n, (n // 1000,), device=device, generator=gen)
    saved = grad[bad].clone()
    grad[bad] = float("inf")
    param.grad = grad
    _, stepped = _engine_step(opt, scaler, param)
    assert not stepped
    assert np.array_equal(param.detach()[idx].cpu().numpy().view(np.int32), P.view(np.int32))
    # Restore finite values; after the backoff the gradient is scaled by 2^15.
    grad[bad] = saved
    grad.mul_(0.5)
    G = _bf16_bits(grad[idx])
    param.grad = grad
    norm, stepped = _engine_step(opt, scaler, param)
    assert stepped
    mul = oracle.clip_multiplier(float(norm), 1.0)
    assert mul < 1.0  # norm ~ sqrt(n) * 1e-4 ~ 9.4
    M = np.zeros(idx.numel(), np.float32)
    V = np.zeros(idx.numel(), np.float32)
    sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=1.0)
    oracle.adamw_step(P, G, M, V, sc, unscale=1.0 / scaler.scale_value, grad_mul=mul)
    assert np.array_equal(param.detach()[idx].cpu().numpy().view(np.int32), P.view(np.int32))
    state = opt.inner.state[param]
    assert np.array_equal(state["exp_avg"][idx].cpu().numpy().view(np.int32), M.view(np.int32))
    del opt, param, grad, state
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name", ["adamw", "sgd"])
def test_bf16_engine_sequence_eager_and_deferred_match_the_oracle(device, name):
    """The engine's tail (``unscale_``, ``clip_grad_norm``, ``scaler.step``, ``update``) on
    bf16 gradients with a loss scale of 1000 (its inverse is not a power of two, so the
    unscale rounds) and a clip coefficient near 0.3 (not a power of two either), run
    three ways: everything in place (the defaults), everything deferred, and a deferred
    unscale under an in-place clip.  Every way gives parameters and state bitwise equal to
    the oracle, whose gradient is rounded to bf16 after each multiply as the reference's
    ``grad.mul_`` calls round it (``optim/grad_scaler.py:181-186``,
    ``optim/sharded_optimizer.py:333-337``), and the in-place ways leave exactly those
    rounded gradients in ``.grad``."""
    n = 300_001
    scale = 1000.0
    gen = torch.Generator(device=device).manual_seed(21)
    p0 = torch.randn(n, device=device, generator=gen) * 0.02
    grads = [(torch.randn(n, device=device, generator=gen) * 3e-3 * scale).to(torch.bfloat16) for _ in range(3)]
    config = (OptimizerConfig(learning_rate=3e-4, betas=(0.9, 0.95), weight_decay=0.1) if name == "adamw"
              else OptimizerConfig(name="sgd", learning_rate=0.05, momentum=0.9, weight_decay=0.01))
    results = {}
    for defer_unscale, defer_clip in ((False, False), (True, True), (True, False)):
        param = torch.nn.Parameter(p0.clone())
        param.grad_dtype = None
        opt = ShardedOptimizer([param], config, norm_group=GroupHandle.trivial(), device=device, defer_clip=defer_clip)
        scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=scale, growth_interval=1000),
                            GroupHandle.trivial(), device, defer_unscale=defer_unscale)
        P = p0.cpu().numpy().copy()
        M = np.zeros(n, np.float32)
        V = np.zeros(n, np.float32)
        for step, g in enumerate(grads, start=1):
            G = _bf16_bits(g)
            param.grad = g.clone()
            scaler.unscale_([param])
            norm = float(opt.clip_grad_norm(1.0))
            assert scaler.step(opt, [param], already_unscaled=True)
            scaler.update()
            ref_sq = oracle.sqnorm(G, unscale=1.0 / scale)
            assert abs(norm**2 - ref_sq) <= 1e-12 * ref_sq
            mul = oracle.clip_multiplier(norm, 1.0)
            assert mul < 1.0 and math.frexp(mul)[0] != 0.5  # clipping active, not a power of two
            written = np.empty(n, np.uint16)
            if name == "adamw":
                sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=float(step))
                oracle.adamw_step(P, G, M, V, sc, unscale=1.0 / scale, grad_mul=mul, grad_out=written)
            else:
                oracle.sgd_step(P, G, M, lr=0.05, momentum=0.9, weight_decay=0.01, first=step == 1,
                                unscale=1.0 / scale, grad_mul=mul, grad_out=written)
            assert np.array_equal(param.detach().cpu().numpy().view(np.int32), P.view(np.int32)), (step, defer_clip)
            state = opt.inner.state[param]
            first = state["exp_avg"] if name == "adamw" else state["momentum_buffer"]
            assert np.array_equal(first.cpu().numpy().view(np.int32), M.view(np.int32)), (step, defer_clip)
            if name == "adamw":
                assert np.array_equal(state["exp_avg_sq"].cpu().numpy().view(np.int32), V.view(np.int32))
            # .grad: the in-place sequence's rounded values, or untouched when both are deferred
            assert np.array_equal(_bf16_bits(param.grad), G if defer_clip else written), (step, defer_clip)
            opt.zero_grad(set_to_none=True)
        results[(defer_unscale, defer_clip)] = param.detach().cpu()
    first = results[(False, False)]
    assert all(torch.equal(first, r) for r in results.values())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_eager_unscale_partials_feed_the_clip_norm(device, monkeypatch, dtype):
    """An eager ``unscale_`` sums the squares of the unscaled values in the same pass that
    writes them (``hbt_scale_inplace_sqnorm``): its overflow check launches no norm
    kernel, the partials stay on the gradients, and ``clip_grad_norm`` on the unchanged
    gradients reads no gradient either; its norm and multiplier are bitwise those of a
    pass over untagged copies.  An in-place change to one gradient drops that gradient's
    partials (its version counter moves), and only that gradient is read again."""
    from hybrid_training_amd import optim as optim_module

    gen = torch.Generator(device=device).manual_seed(33)
    sizes = [100_003, 70_000, 1]
    params = [torch.nn.Parameter(torch.randn(n, device=device, generator=gen)) for n in sizes]
    for p in params:
        p.grad_dtype = None
        p.grad = (torch.randn(p.numel(), device=device, generator=gen) * 1000.0).to(dtype)
    copies = [torch.nn.Parameter(p.detach().clone()) for p in params]
    # the clip is left to the step, so the gradients stay as the unscale wrote them
    opt = ShardedOptimizer(params, OptimizerConfig(), norm_group=GroupHandle.trivial(), device=device,
                           clip_in_step=True)
    scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=1000.0), GroupHandle.trivial(), device)
    launched = []
    real = optim_module._launch_sqnorm

    def counting(lib, items, *args):
        launched.extend(g.numel() for g, _, _, _ in items)
        return real(lib, items, *args)

    monkeypatch.setattr(optim_module, "_launch_sqnorm", counting)
    assert not scaler.unscale_(params)
    assert launched == []  # the overflow check read the fused pass's partials
    for c, p in zip(copies, params):
        c.grad_dtype = None
        c.grad = p.grad.clone()  # the unscaled values, without partials attached
    norm = opt.clip_grad_norm(1.0)
    assert launched == []  # every segment came from the scaler's partials
    ref_opt = ShardedOptimizer(copies, OptimizerConfig(), norm_group=GroupHandle.trivial(), device=device,
                               clip_in_step=True)
    ref = ref_opt.clip_grad_norm(1.0)
    assert sorted(launched) == sorted(sizes)  # the copies were read
    assert float(norm) == float(ref)  # the clip multiplier is derived from the same fp64 sum
    launched.clear()
    params[1].grad.mul_(1.0)  # an in-place op: the version counter moves
    # a fresh optimizer (the first one holds a pending clip, which refuses changed gradients)
    again = ShardedOptimizer(params, OptimizerConfig(), norm_group=GroupHandle.trivial(), device=device)
    assert float(again.clip_grad_norm(1.0)) == float(ref)
    assert launched == [sizes[1]]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_unscale_twice_before_a_step_multiplies_twice(device, dtype):
    """Two ``unscale_`` calls with no step between them multiply twice, as the
    reference's two ``grad.mul_(inverse)`` do (``grad_scaler.py:181-186``).  The eager
    result is torch's own pair of in-place multiplies, bitwise; with ``defer_unscale``
    the factor still pending from the first call is applied before the second is
    deferred, so after the clipped step ``.grad``, the parameters and the norm are
    bitwise the eager sequence's."""
    n = 200_003
    gen = torch.Generator(device=device).manual_seed(41)
    p0 = torch.randn(n, device=device, generator=gen) * 0.02
    g = (torch.randn(n, device=device, generator=gen) * 1e-3 * 1000.0).to(dtype)
    inverse = 1.0 / 1000.0
    twice = g.clone().mul_(inverse).mul_(inverse)
    results = []
    for defer in (False, True):
        param = torch.nn.Parameter(p0.clone())
        param.grad_dtype = None
        opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=3e-4, weight_decay=0.1),
                               norm_group=GroupHandle.trivial(), device=device)
        scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=1000.0), GroupHandle.trivial(), device,
                            defer_unscale=defer)
        param.grad = g.clone()
        assert not scaler.unscale_([param])
        assert not scaler.unscale_([param])
        if not defer:
            assert torch.equal(param.grad.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                               twice.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
        norm = opt.clip_grad_norm(1e-3)
        assert scaler.step(opt, [param], already_unscaled=True)
        results.append((param.detach().clone(), param.grad.detach().clone(), float(norm)))
    (p_e, g_e, n_e), (p_d, g_d, n_d) = results
    assert n_e == n_d
    assert torch.equal(p_e.view(torch.int32), p_d.view(torch.int32))
    bits = torch.int16 if dtype == torch.bfloat16 else torch.int32
    assert torch.equal(g_e.view(bits), g_d.view(bits))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("finite", [True, False])
def test_deferred_unscale_with_a_plain_torch_optimizer(device, dtype, finite):
    """The reference's ``GradScaler.step`` takes any optimizer with a ``step()``, a plain
    ``torch.optim.Optimizer`` included (``grad_scaler.py:202-241``).  Only
    ``ShardedOptimizer`` applies a deferred unscale while it reads the gradient, so for
    any other optimizer ``step`` applies it in place first, stepped or skipped: the plain
    optimizer sees, and ``.grad`` keeps, exactly the eager unscale's gradient, which is
    torch's ``grad.mul_(1 / scale)`` followed by torch's own SGD step."""
    n = 100_003
    gen = torch.Generator(device=device).manual_seed(43)
    p0 = (torch.randn(n, device=device, generator=gen) * 0.02).to(dtype)
    g = (torch.randn(n, device=device, generator=gen) * 1e-3 * SCALE).to(dtype)
    if not finite:
        g[77] = float("inf")
    results = []
    for defer in (False, True, None):
        param = torch.nn.Parameter(p0.clone())
        plain = torch.optim.SGD([param], lr=0.1, momentum=0.9)
        param.grad = g.clone()
        if defer is None:  # the reference's sequence in torch ops
            param.grad.mul_(1.0 / SCALE)
            stepped = bool(torch.isfinite(param.grad).all())
            if stepped:
                plain.step()
        else:
            scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=SCALE), GroupHandle.trivial(), device,
                                defer_unscale=defer)
            stepped = scaler.step(plain, [param])
        assert stepped == finite
        results.append((param.detach().clone(), param.grad.detach().clone()))
    bits = torch.int16 if dtype == torch.bfloat16 else torch.int32
    for p, gr in results[:2]:
        assert torch.equal(p.view(bits), results[2][0].view(bits))
        assert torch.equal(gr.view(bits), results[2][1].view(bits))
