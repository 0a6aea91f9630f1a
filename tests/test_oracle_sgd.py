"""The SGD restatement of the oracle against torch.optim.SGD on CPU tensors.

The reference builds ``torch.optim.SGD(params, lr, momentum, weight_decay)``
(``optim/sharded_optimizer.py:121-126``); on CPU tensors it runs
``_single_tensor_sgd``.  The oracle must match it bitwise over several steps, for
every combination of momentum, weight decay, dampening and Nesterov, and reduce to
the closed form ``p - lr * g`` for a plain step.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle


@pytest.mark.parametrize("momentum,dampening,nesterov", [(0.0, 0.0, False), (0.9, 0.0, False),
                                                         (0.9, 0.1, False), (0.9, 0.0, True)])
@pytest.mark.parametrize("weight_decay", [0.0, 0.01])
def test_bitwise_with_torch_sgd(momentum, dampening, nesterov, weight_decay):
    n, lr = 10_007, 0.05
    gen = torch.Generator().manual_seed(7)
    param = torch.nn.Parameter(torch.randn(n, generator=gen))
    opt = torch.optim.SGD([param], lr=lr, momentum=momentum, dampening=dampening, nesterov=nesterov,
                          weight_decay=weight_decay, foreach=False)
    p = param.detach().numpy().copy()
    buf = np.zeros(n, np.float32) if momentum else None
    for step in range(4):
        g = torch.randn(n, generator=gen) * 0.1
        param.grad = g.clone()
        opt.step()
        oracle.sgd_step(p, g.numpy(), buf, lr=lr, momentum=momentum, dampening=dampening,
                        weight_decay=weight_decay, nesterov=nesterov, first=step == 0)
        assert np.array_equal(param.detach().numpy().view(np.int32), p.view(np.int32)), step
        if momentum:
            assert np.array_equal(opt.state[param]["momentum_buffer"].numpy().view(np.int32), buf.view(np.int32))


def test_plain_step_closed_form():
    p = np.array([1.0, -2.0, 0.5], np.float32)
    g = np.array([0.25, 1.0, -4.0], np.float32)
    oracle.sgd_step(p, g, None, lr=0.5)
    assert p.tolist() == [0.875, -2.5, 2.5]


def test_clip_and_unscale_multiplies_come_first():
    rng = np.random.default_rng(3)
    g = rng.standard_normal(1000).astype(np.float32) * 65536
    p0 = rng.standard_normal(1000).astype(np.float32)
    a, b = p0.copy(), p0.copy()
    oracle.sgd_step(a, g, None, lr=0.1, weight_decay=0.01, unscale=1 / 65536, grad_mul=0.3)
    scaled = ((g * np.float32(1 / 65536)).astype(np.float32) * np.float32(0.3)).astype(np.float32)
    oracle.sgd_step(b, scaled, None, lr=0.1, weight_decay=0.01)
    assert np.array_equal(a, b)
