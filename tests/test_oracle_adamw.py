"""Pins the oracle's AdamW restatement to torch.optim.AdamW on the CPU.

The reference does no AdamW arithmetic of its own: ``optim/sharded_optimizer.py:111-120``
builds ``torch.optim.AdamW`` and ``:355`` calls its ``step()``, which on CPU tensors
runs ``_single_tensor_adam`` (``torch/optim/adam.py:396-547``).  So torch itself is
the library routine the oracle must reproduce.

* With torch's own ``exp_avg_sq.sqrt()`` injected, the oracle must match torch
  BITWISE in p, m and v at every step.  That pins every other operation (the decay
  multiply, the fused lerp, the fused addcmul, both divisions, the add, the clip
  multiply) and the host scalars.
* With its own correctly rounded sqrtf, the oracle may differ from torch where
  torch's vectorised sqrt is not correctly rounded (it routes large tensors
  through a faithfully rounded library sqrt).  That difference is bounded
  element-wise by ``|a - b| <= 1e-6 * max(|b|, lr)``.
* Step 1 from zero state has a closed form: m = (1-b1) g, v = (1-b2) g^2 up to
  rounding, and the update is -lr * g / (|g| + eps) up to rounding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

#: Tolerance of the oracle (correctly rounded sqrt) against torch's CPU AdamW:
#: relative 1e-6, with the learning rate as the magnitude floor (an element near
#: zero is compared at the scale of one update).
RTOL = 1e-6


def _run_pair(n, steps, lr, betas, eps, wd, clip, seed, inject_sqrt):
    gen = torch.Generator().manual_seed(seed)
    p0 = torch.randn(n, generator=gen) * 0.02
    param = torch.nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([param], lr=lr, betas=betas, eps=eps, weight_decay=wd, foreach=False)
    p = p0.clone().numpy()
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    for step in range(1, steps + 1):
        g = torch.randn(n, generator=gen) * 1e-2
        grad = g.clone()
        if clip != 1.0:
            grad.mul_(clip)  # the reference's clip: grad.mul_(python float)
        param.grad = grad
        opt.step()
        state = opt.state[param]
        scalars = oracle.adamw_scalars(
            lr=lr, beta1=betas[0], beta2=betas[1], eps=eps, weight_decay=wd, step=float(step)
        )
        root = state["exp_avg_sq"].sqrt().numpy() if inject_sqrt else None
        oracle.adamw_step(p, g.numpy(), m, v, scalars, grad_mul=float(np.float32(clip)),
                          sqrt_override=root)
        yield step, param.detach().numpy(), state["exp_avg"].numpy(), state["exp_avg_sq"].numpy(), p, m, v


@pytest.mark.parametrize(
    ("n", "steps", "lr", "betas", "wd", "clip"),
    [
        (65_537, 10, 3e-4, (0.9, 0.95), 0.1, 0.3157),  # the Llama shard's hyper-parameters
        (1857, 5, 1e-3, (0.9, 0.999), 0.01, 1.0),  # the 1857-parameter MLP's
        (333, 4, 1e-2, (0.3, 0.9), 0.0, 0.5),  # lerp weight 0.7: the other lerp branch
    ],
)
def test_bitwise_with_torch_sqrt(n, steps, lr, betas, wd, clip):
    for step, tp, tm, tv, p, m, v in _run_pair(n, steps, lr, betas, 1e-8, wd, clip, 7, True):
        assert np.array_equal(tm, m), f"exp_avg differs at step {step}"
        assert np.array_equal(tv, v), f"exp_avg_sq differs at step {step}"
        assert np.array_equal(tp, p), f"param differs at step {step}"


def test_within_tolerance_with_own_sqrt():
    lr = 3e-4
    worst = 0.0
    for _, tp, tm, tv, p, m, v in _run_pair(1 << 18, 10, lr, (0.9, 0.95), 1e-8, 0.1, 0.3, 3, False):
        assert np.array_equal(tm, m) and np.array_equal(tv, v)
        worst = max(worst, float(np.max(np.abs(tp - p) / np.maximum(np.abs(tp), lr))))
    assert worst <= RTOL, worst


def test_first_step_closed_form():
    n = 4096
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    p = np.zeros(n, np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    oracle.adamw_step(p, g, m, v, oracle.adamw_scalars(lr=lr, beta1=b1, beta2=b2, eps=eps,
                                                       weight_decay=0.0, step=1.0))
    np.testing.assert_allclose(m, (1 - b1) * g.astype(np.float64), rtol=1e-6)
    np.testing.assert_allclose(v, (1 - b2) * g.astype(np.float64) ** 2, rtol=1e-6)
    expected = -lr * g.astype(np.float64) / (np.abs(g.astype(np.float64)) + eps)
    np.testing.assert_allclose(p, expected, rtol=1e-5)


def test_weight_decay_only_step_is_a_pure_decay():
    # g = 0 and zero state: the update term is 0 / (0 + eps) = 0, so p = fp32(p * (1 - lr*wd)).
    p = np.linspace(-1, 1, 101, dtype=np.float32)
    expect = (p * np.float32(1 - 1e-2 * 0.1)).astype(np.float32)
    oracle.adamw_step(p, np.zeros_like(p), np.zeros_like(p), np.zeros_like(p),
                      oracle.adamw_scalars(lr=1e-2, beta1=0.9, beta2=0.999, eps=1e-8,
                                           weight_decay=0.1, step=1.0))
    assert np.array_equal(p, expect)


def test_bf16_gradient_widening_matches_fp32_path():
    rng = np.random.default_rng(9)
    g32 = (rng.standard_normal(999) * 1e-2).astype(np.float32)
    g16 = oracle.f32_to_bf16(g32)
    widened = (g16.astype(np.uint32) << 16).view(np.float32)
    sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=1.0)
    p1 = (rng.standard_normal(999) * 0.02).astype(np.float32)
    p2, m1, m2, v1, v2 = p1.copy(), *(np.zeros(999, np.float32) for _ in range(4))
    oracle.adamw_step(p1, g16, m1, v1, sc, unscale=2.0**-16)
    oracle.adamw_step(p2, widened, m2, v2, sc, unscale=2.0**-16)
    assert np.array_equal(p1, p2) and np.array_equal(m1, m2) and np.array_equal(v1, v2)
