"""GPU parity of the fused clip + SGD step (``hbt_sgd_step``).

The reference's second inner optimizer is ``torch.optim.SGD(params, lr, momentum,
weight_decay)`` (``optim/sharded_optimizer.py:121-126``).  ``ShardedOptimizer`` with
``OptimizerConfig(name="sgd")`` must leave parameters and momentum buffers bitwise
equal to the oracle (itself bitwise equal to torch's CPU SGD) over several steps, with
and without momentum, weight decay, dampening and Nesterov, for aligned, misaligned
and tail-sized tensors, more than 16 tensors per step, fp32 and bf16 gradients, and
with the deferred clip and loss-scale multiplies.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import GradScaler, GradScalerConfig, GroupHandle, OptimizerConfig, ShardedOptimizer

pytestmark = pytest.mark.gpu


def _i32(a):
    return np.ascontiguousarray(a).view(np.int32)


@pytest.mark.parametrize("momentum,dampening,nesterov", [(0.0, 0.0, False), (0.9, 0.0, False),
                                                         (0.9, 0.25, False), (0.9, 0.0, True)])
@pytest.mark.parametrize("weight_decay", [0.0, 0.01])
def test_sgd_matches_oracle(device, momentum, dampening, nesterov, weight_decay):
    lr = 0.05
    sizes = [100_003, 512, 511, 1, 4096] + [257] * 14  # 19 tensors: two launches
    gen = torch.Generator(device=device).manual_seed(11)
    storage = torch.randn(sum(sizes) + 1, device=device, generator=gen)
    params, cursor = [], 1  # the first tensor starts one element in: misaligned
    for n in sizes:
        params.append(torch.nn.Parameter(storage[cursor : cursor + n].clone() if n != 100_003
                                         else storage[cursor : cursor + n]))
        cursor += n
    opt = ShardedOptimizer(params, OptimizerConfig(name="sgd", learning_rate=lr, momentum=momentum,
                                                   weight_decay=weight_decay),
                           norm_group=GroupHandle.trivial(), device=device)
    for group in opt.inner.param_groups:
        group["dampening"] = dampening
        group["nesterov"] = nesterov
    host_p = [p.detach().cpu().numpy().copy() for p in params]
    host_b = [np.zeros(p.numel(), np.float32) for p in params] if momentum else [None] * len(params)
    for step in range(3):
        grads = [torch.randn(p.shape, device=device, generator=gen) * 0.1 for p in params]
        for p, g in zip(params, grads):
            p.grad = g
        opt.step()
        for hp, hb, g in zip(host_p, host_b, grads):
            oracle.sgd_step(hp, g.cpu().numpy(), hb, lr=lr, momentum=momentum, dampening=dampening,
                            weight_decay=weight_decay, nesterov=nesterov, first=step == 0)
        for p, hp in zip(params, host_p):
            assert np.array_equal(_i32(p.detach().cpu().numpy()), _i32(hp)), step
        if momentum:
            for p, hb in zip(params, host_b):
                assert np.array_equal(_i32(opt.inner.state[p]["momentum_buffer"].cpu().numpy()), _i32(hb))
        else:
            assert all(len(opt.inner.state[p]) == 0 for p in params)


def test_sgd_with_deferred_clip_and_bf16_loss_scaled_grads(device):
    n, lr, scale = 300_007, 0.02, 65536.0
    gen = torch.Generator(device=device).manual_seed(12)
    param = torch.nn.Parameter(torch.randn(n, device=device, generator=gen))
    param.grad_dtype = None
    opt = ShardedOptimizer([param], OptimizerConfig(name="sgd", learning_rate=lr, momentum=0.9, weight_decay=0.01),
                           norm_group=GroupHandle.trivial(), device=device, defer_clip=True)
    scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=scale), GroupHandle.trivial(), device,
                        defer_unscale=True)
    hp = param.detach().cpu().numpy().copy()
    hb = np.zeros(n, np.float32)
    for step in range(3):
        g = (torch.randn(n, device=device, generator=gen) * (0.05 * scale)).to(torch.bfloat16)
        param.grad = g
        scaler.unscale_([param])
        norm = float(opt.clip_grad_norm(1.0))
        assert scaler.step(opt, [param], already_unscaled=True)
        scaler.update()
        opt.zero_grad()
        bits = g.cpu().view(torch.int16).numpy().view(np.uint16)
        ref = oracle.sqnorm(bits, unscale=1.0 / scale)
        assert abs(norm**2 - ref) <= 1e-12 * ref
        mul = oracle.clip_multiplier(norm, 1.0)
        assert mul < 1.0
        # the unscale and clip multiplies are each rounded to bf16, as the reference's
        # in-place grad.mul_ calls on a bf16 gradient round them
        oracle.sgd_step(hp, bits, hb, lr=lr, momentum=0.9, weight_decay=0.01, first=step == 0,
                        unscale=1.0 / scale, grad_mul=mul)
        assert np.array_equal(_i32(param.detach().cpu().numpy()), _i32(hp)), step


def test_sgd_state_dict_round_trip(device):
    params = [torch.nn.Parameter(torch.randn(1000, device=device)) for _ in range(3)]
    opt = ShardedOptimizer(params, OptimizerConfig(name="sgd", learning_rate=0.1, momentum=0.9),
                           norm_group=GroupHandle.trivial(), device=device)
    for p in params:
        p.grad = torch.randn_like(p)
    opt.step()
    saved = opt.state_dict()
    fresh = ShardedOptimizer(params, OptimizerConfig(name="sgd", learning_rate=0.1, momentum=0.9),
                             norm_group=GroupHandle.trivial(), device=device)
    fresh.load_state_dict(saved)
    for p in params:
        assert torch.equal(fresh.inner.state[p]["momentum_buffer"], opt.inner.state[p]["momentum_buffer"])
    assert fresh.state_bytes() == opt.state_bytes() == 3 * 1000 * 4


@pytest.mark.parametrize("nesterov", [False, True])
def test_sgd_with_ieee_specials_matches_oracle(device, nesterov):
    """IEEE specials through the fused SGD update over two steps (the buffer's first write,
    then the momentum update): gradients ±inf, NaN, -0.0, the largest finite value and a
    denormal, parameters -0.0 and NaN, in the vector body and the tail; every non-NaN
    parameter and buffer element bitwise the oracle's, NaNs in the same places."""
    n, lr = 4096 + 29, 0.05
    gen = torch.Generator(device=device).manual_seed(73)
    p0 = torch.randn(n, device=device, generator=gen)
    for base in (0, 4096):
        p0[base + 6] = -0.0
        p0[base + 7] = float("nan")
    param = torch.nn.Parameter(p0.clone())
    opt = ShardedOptimizer([param], OptimizerConfig(name="sgd", learning_rate=lr, momentum=0.9, weight_decay=0.01),
                           norm_group=GroupHandle.trivial(), device=device)
    for group in opt.inner.param_groups:
        group["nesterov"] = nesterov
    hp, hb = p0.cpu().numpy().copy(), np.zeros(n, np.float32)
    for step in range(2):
        g = torch.randn(n, device=device, generator=gen) * 0.1
        for base in (0, 4096):
            g[base + 0] = float("inf")
            g[base + 1] = -float("inf")
            g[base + 2] = float("nan")
            g[base + 3] = -0.0
            g[base + 4] = torch.finfo(torch.float32).max
            g[base + 5] = 1e-40
        param.grad = g
        opt.step()
        oracle.sgd_step(hp, g.cpu().numpy(), hb, lr=lr, momentum=0.9, weight_decay=0.01, nesterov=nesterov,
                        first=step == 0)
        for got, want in ((param.detach().cpu().numpy(), hp), (opt.inner.state[param]["momentum_buffer"].cpu().numpy(), hb)):
            nan = np.isnan(want)
            assert np.array_equal(np.isnan(got), nan), step
            assert np.array_equal(_i32(got[~nan]), _i32(want[~nan])), step
