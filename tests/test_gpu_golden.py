"""The HIP path against the committed golden vectors (torch.optim.AdamW on CPU).

Drives the drop-in ``ShardedOptimizer`` with the golden inputs: m and v must equal
torch's bitwise, p must be within ``|a - b| <= 1e-6 * max(|b|, lr)``, and every
tensor must equal the oracle's bitwise.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import GroupHandle, OptimizerConfig, ShardedOptimizer

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RTOL = 1e-6


def _rel(a, b, floor):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), floor)))


@pytest.mark.parametrize("defer", [False, True])
def test_clipped_adamw_trajectory(device, defer):
    g = np.load(os.path.join(GOLDEN, "adamw_llama_shard_4096.npz"))
    lr, b1, b2, eps, wd, max_norm = (float(x) for x in g["hyper"])
    param = torch.nn.Parameter(torch.from_numpy(g["p0"].copy()).to(device))
    opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=lr, betas=(b1, b2), eps=eps, weight_decay=wd),
                           norm_group=GroupHandle.trivial(), device=device, defer_clip=defer)
    p, m, v = g["p0"].copy(), np.zeros(4096, np.float32), np.zeros(4096, np.float32)
    for k in range(g["grads"].shape[0]):
        param.grad = torch.from_numpy(g["grads"][k].copy()).to(device)
        norm = float(opt.clip_grad_norm(max_norm))
        assert abs(norm - g["norms"][k]) <= 1e-12 * g["norms"][k]
        opt.step()
        opt.zero_grad()
        sc = oracle.adamw_scalars(lr=lr, beta1=b1, beta2=b2, eps=eps, weight_decay=wd, step=float(k + 1))
        oracle.adamw_step(p, g["grads"][k], m, v, sc, grad_mul=oracle.clip_multiplier(norm, max_norm))
    state = opt.inner.state[param]
    got_p = param.detach().cpu().numpy()
    assert np.array_equal(state["exp_avg"].cpu().numpy(), g["m"])
    assert np.array_equal(state["exp_avg_sq"].cpu().numpy(), g["v"])
    assert _rel(got_p, g["p"], lr) <= RTOL
    assert np.array_equal(got_p.view(np.int32), p.view(np.int32))


def test_fsdp_mlp_shards(device):
    g = np.load(os.path.join(GOLDEN, "fsdp_mlp_1857.npz"))
    for world in (2, 4):
        params = [torch.nn.Parameter(torch.from_numpy(s.copy()).to(device)) for s in g[f"w{world}_initial"]]
        opts = [ShardedOptimizer([p], OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                                 norm_group=GroupHandle.local_view("world", world, r), device=device)
                for r, p in enumerate(params)]
        for step in range(5):
            for r, (p, opt) in enumerate(zip(params, opts)):
                p.grad = torch.from_numpy(g[f"w{world}_grads"][step, r].copy()).to(device)
                opt.step()
            got = np.stack([p.detach().cpu().numpy() for p in params])
            assert _rel(got, g[f"w{world}_shards"][step], 1e-3) <= RTOL
