"""Pins the float64 restatements to torch's optimizers stepping float64 CPU tensors.

With mixed precision off the reference's masters, gradients and optimizer state are the
parameters' own dtype (``parallel/fsdp.py:379-393``), and ``torch.optim.AdamW`` / ``SGD``
(``optim/sharded_optimizer.py:111-126``) step them with every Python scalar used as the
double it is.  torch is the library routine the oracle must reproduce:

* ``adamw_step_f64`` equals torch's AdamW bitwise in p, m and v at every step when
  torch's own ``exp_avg_sq.sqrt()`` is injected, on both branches of the lerp, with and
  without weight decay and a clip multiply (torch's own ``grad.mul_(coefficient)`` in the
  reference's order), and from step 1's closed form.  torch's float64 CPU sqrt is not
  correctly rounded on large tensors (about 1 element in 130 differs from the correctly
  rounded root at the Llama shard's statistics); with its own correctly rounded sqrt,
  as the kernels compute, m and v stay bitwise and p is within 1e-15 relative;
* the same restatement with the addcmul product rounded before the add (a plausible
  slip) is not torch's, so the comparison can tell the two apart;
* ``sgd_step_f64`` equals torch's SGD bitwise for every combination of momentum,
  dampening, weight decay and Nesterov;
* ``sqnorm_f64`` is the correctly rounded sum of the rounded double squares (``math.fsum``)
  and agrees with torch's ``pow(2).sum()``.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

import oracle


def _torch_adamw_pair(n, steps, lr, betas, wd, clip, seed, inject_sqrt=True):
    gen = torch.Generator().manual_seed(seed)
    p0 = torch.randn(n, generator=gen, dtype=torch.float64) * 0.02
    param = torch.nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([param], lr=lr, betas=betas, eps=1e-8, weight_decay=wd, foreach=False)
    p = p0.numpy().copy()
    m = np.zeros(n)
    v = np.zeros(n)
    for step in range(1, steps + 1):
        g = torch.randn(n, generator=gen, dtype=torch.float64) * 1e-2
        grad = g.clone()
        mul = 1.0
        if clip is not None:
            norm = float(grad.pow(2).sum().sqrt())
            mul = oracle.clip_multiplier64(norm, clip)
            if mul < 1.0:
                grad.mul_(max(clip, 0.0) / (norm + 1e-6))  # the reference's grad.mul_(coefficient)
        param.grad = grad
        opt.step()
        scalars = oracle.adamw_scalars(lr=lr, beta1=betas[0], beta2=betas[1], eps=1e-8, weight_decay=wd,
                                       step=float(step))
        state = opt.state[param]
        root = state["exp_avg_sq"].sqrt().numpy() if inject_sqrt else None
        oracle.adamw_step_f64(p, g.numpy(), m, v, scalars, grad_mul=mul, sqrt_override=root)
        yield step, param.detach().numpy(), state["exp_avg"].numpy(), state["exp_avg_sq"].numpy(), p, m, v


@pytest.mark.parametrize(
    ("n", "steps", "lr", "betas", "wd", "clip"),
    [
        (65_537, 10, 3e-4, (0.9, 0.95), 0.1, 1.0),  # the Llama shard's hyper-parameters, clip active
        (1857, 5, 1e-3, (0.9, 0.999), 0.01, None),  # the 1857-parameter MLP's, no clip
        (333, 4, 1e-2, (0.3, 0.9), 0.0, 0.05),  # lerp weight 0.7: the other branch; no decay
    ],
)
def test_adamw_f64_is_torch_bitwise(n, steps, lr, betas, wd, clip):
    for step, tp, tm, tv, p, m, v in _torch_adamw_pair(n, steps, lr, betas, wd, clip, 11):
        assert np.array_equal(tm, m), f"exp_avg differs at step {step}"
        assert np.array_equal(tv, v), f"exp_avg_sq differs at step {step}"
        assert np.array_equal(tp, p), f"param differs at step {step}"


def test_adamw_f64_with_its_own_sqrt_is_within_1e15():
    worst = 0.0
    for _, tp, tm, tv, p, m, v in _torch_adamw_pair(1 << 17, 10, 3e-4, (0.9, 0.95), 0.1, 1.0, 4, inject_sqrt=False):
        assert np.array_equal(tm, m) and np.array_equal(tv, v)
        worst = max(worst, float(np.max(np.abs(tp - p) / np.maximum(np.abs(tp), 3e-4))))
    assert worst <= 1e-15, worst


def test_a_rounded_addcmul_product_is_not_torch():
    """The second moment with its product rounded before the add, (c*g)*g + v in three
    roundings, differs from torch on a random shard: the comparison above would catch it."""
    n = 4099
    gen = torch.Generator().manual_seed(3)
    param = torch.nn.Parameter(torch.zeros(n, dtype=torch.float64))
    opt = torch.optim.AdamW([param], lr=1e-3, betas=(0.9, 0.95), weight_decay=0.0, foreach=False)
    v = np.zeros(n)
    for _ in range(3):
        g = torch.randn(n, generator=gen, dtype=torch.float64)
        param.grad = g.clone()
        opt.step()
        x = g.numpy()
        v = v * 0.95 + ((1 - 0.95) * x) * x  # the slip
    assert not np.array_equal(opt.state[param]["exp_avg_sq"].numpy(), v)


def test_adamw_f64_first_step_closed_form():
    rng = np.random.default_rng(5)
    g = rng.standard_normal(4096) * 1e-3
    p, m, v = np.zeros(4096), np.zeros(4096), np.zeros(4096)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    oracle.adamw_step_f64(p, g, m, v, oracle.adamw_scalars(lr=lr, beta1=b1, beta2=b2, eps=eps, weight_decay=0.0,
                                                            step=1.0))
    np.testing.assert_allclose(m, (1 - b1) * g, rtol=1e-15)
    np.testing.assert_allclose(v, (1 - b2) * g * g, rtol=1e-15)
    np.testing.assert_allclose(p, -lr * g / (np.abs(g) + eps), rtol=1e-12)


@pytest.mark.parametrize("momentum, dampening, wd, nesterov",
                         [c for c in itertools.product((0.0, 0.9), (0.0, 0.1), (0.0, 0.01), (False, True))
                          if not (c[3] and (c[0] == 0.0 or c[1] != 0.0))])
def test_sgd_f64_is_torch_bitwise(momentum, dampening, wd, nesterov):
    n = 10_007
    gen = torch.Generator().manual_seed(17)
    p0 = torch.randn(n, generator=gen, dtype=torch.float64)
    param = torch.nn.Parameter(p0.clone())
    opt = torch.optim.SGD([param], lr=0.05, momentum=momentum, dampening=dampening, weight_decay=wd,
                          nesterov=nesterov, foreach=False)
    p = p0.numpy().copy()
    buf = np.zeros(n)
    for step in range(4):
        g = torch.randn(n, generator=gen, dtype=torch.float64) * 0.1
        param.grad = g.clone()
        opt.step()
        oracle.sgd_step_f64(p, g.numpy(), buf, lr=0.05, momentum=momentum, dampening=dampening, weight_decay=wd,
                            nesterov=nesterov, first=step == 0)
        assert np.array_equal(param.detach().numpy(), p), step
        if momentum:
            assert np.array_equal(opt.state[param]["momentum_buffer"].numpy(), buf), step


def test_sqnorm_f64_is_the_correctly_rounded_sum_of_squares():
    rng = np.random.default_rng(2)
    for scale in (1e-3, 1.0, 1e150):
        g = rng.standard_normal(20_011) * scale
        exact = math.fsum([float(x) * float(x) for x in g])
        assert oracle.sqnorm_f64(g) == exact
        torch_sum = float(torch.from_numpy(g).pow(2).sum())
        assert abs(torch_sum - exact) <= 1e-13 * exact
    assert oracle.sqnorm_f64(np.array([3.0, 4.0])) == 25.0
    assert math.isinf(oracle.sqnorm_f64(np.array([1e200, 1.0])))


def test_clip_multiplier64_is_the_python_double():
    assert oracle.clip_multiplier64(6.0, 1.0) == 1.0 / (6.0 + 1e-6)
    assert oracle.clip_multiplier64(0.5, 1.0) == 1.0
    assert oracle.clip_multiplier64(6.0, 0.0) == 1.0
    g = torch.randn(1000, dtype=torch.float64)
    coef = 1.0 / (6.0 + 1e-6)
    assert torch.equal(g.clone().mul_(coef), torch.from_numpy(g.numpy() * oracle.clip_multiplier64(6.0, 1.0)))
