"""Writes the golden vectors under tests/golden/ (run with the CPU build of torch).

Nothing here imports the reference.  The vectors are produced by the library routine
the reference delegates its optimizer arithmetic to, ``torch.optim.AdamW`` on CPU
tensors (``optim/sharded_optimizer.py:111-120`` builds it, ``:355`` steps it), driven
by the reference's own clip sequence (``optim/sharded_optimizer.py:151-158``,
``:236-241``, ``:331-337``: fp64 squares, sum, sqrt, Python-double coefficient,
``grad.mul_``), and by plain arithmetic for the layout tables.

Files:
  adamw_llama_shard_4096.npz  10 clipped AdamW steps on a 4096-element slice of the
                              Llama-3-8B W=8 shard workload (lr 3e-4, betas (0.9, 0.95),
                              eps 1e-8, weight decay 0.1, clip 1.0)
  fsdp_mlp_1857.npz           the 1857-parameter MLP, W=2 and W=4: every rank's
                              averaged gradient shard for 5 steps and torch AdamW's
                              shard after each step (lr 1e-3, weight decay 0.01)
  layouts.json                GPT-2-small bucket table, shard sizes of the benchmark
                              models, the 4-writer / 3-reader intersection table
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch
import torch.nn as nn

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.model_shapes import GPT2_SMALL, LLAMA3_8B, LLAMA3_70B_TOTAL  # noqa: E402


def _numel(shape):
    n = 1
    for s in shape:
        n *= s
    return n


def adamw_llama_shard() -> None:
    n, steps, max_norm = 4096, 10, 1.0
    gen = torch.Generator().manual_seed(20260101)
    p0 = torch.randn(n, generator=gen) * 0.02
    # The full shard's norm is ~3.17 at g ~ N(0, 1e-4); this slice is scaled so the
    # clip is active at a comparable coefficient.
    grads = torch.randn(steps, n, generator=gen) * 0.05
    param = nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([param], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, foreach=False)
    norms, muls = [], []
    for k in range(steps):
        param.grad = grads[k].clone()
        squared = param.grad.detach().to(torch.float64).pow(2).sum()
        norm = float(squared.reshape(1)[0].clamp_min(0).sqrt())
        coef = max_norm / (norm + 1e-6)
        if coef < 1.0:
            param.grad.detach().mul_(coef)
        opt.step()
        norms.append(norm)
        muls.append(coef)
    state = opt.state[param]
    np.savez_compressed(
        os.path.join(HERE, "adamw_llama_shard_4096.npz"),
        p0=p0.numpy(), grads=grads.numpy(), norms=np.array(norms), coefs=np.array(muls),
        p=param.detach().numpy(), m=state["exp_avg"].numpy(), v=state["exp_avg_sq"].numpy(),
        hyper=np.array([3e-4, 0.9, 0.95, 1e-8, 0.1, max_norm]),
    )


def fsdp_mlp() -> None:
    out = {}
    for world in (2, 4):
        torch.manual_seed(3)
        model = nn.Sequential(nn.Linear(23, 32), nn.ReLU(), nn.Linear(32, 32), nn.ReLU(), nn.Linear(32, 1))
        params = list(model.parameters())
        total = sum(p.numel() for p in params)
        shard = -(-total // world)
        flat = torch.zeros(shard * world)
        flat[:total] = torch.cat([p.detach().reshape(-1) for p in params])
        shards = [nn.Parameter(flat[r * shard : (r + 1) * shard].clone()) for r in range(world)]
        opts = [torch.optim.AdamW([s], lr=1e-3, weight_decay=0.01, foreach=False) for s in shards]
        initial = np.stack([s.detach().numpy().copy() for s in shards])
        gen = torch.Generator().manual_seed(11)
        x = torch.randn(5 * world * 16, 23, generator=gen)
        y = torch.randn(5 * world * 16, 1, generator=gen)
        grad_shards, after = [], []
        for step in range(5):
            full_grads = []
            for r in range(world):
                rows = slice((step * world + r) * 16, (step * world + r + 1) * 16)
                model.zero_grad(set_to_none=True)
                nn.functional.mse_loss(model(x[rows]), y[rows]).backward()
                g = torch.zeros(shard * world)
                g[:total] = torch.cat([p.grad.reshape(-1) for p in params])
                full_grads.append(g.div(world))  # AVG pre-divide (collectives.py:593-594)
            summed = full_grads[0].clone()
            for g in full_grads[1:]:
                summed += g  # the reduce-scatter's sum, in rank order
            summed[total:] = 0.0  # _zero_padding_region
            step_grads = []
            for r in range(world):
                shards[r].grad = summed[r * shard : (r + 1) * shard].clone()
                step_grads.append(shards[r].grad.numpy().copy())
                opts[r].step()
            grad_shards.append(np.stack(step_grads))
            after.append(np.stack([s.detach().numpy().copy() for s in shards]))
            with torch.no_grad():
                flat = torch.cat([s.detach() for s in shards])[:total]
                cursor = 0
                for p in params:
                    p.copy_(flat[cursor : cursor + p.numel()].view(p.shape))
                    cursor += p.numel()
        out[f"w{world}_initial"] = initial
        out[f"w{world}_grads"] = np.stack(grad_shards)
        out[f"w{world}_shards"] = np.stack(after)
    np.savez_compressed(os.path.join(HERE, "fsdp_mlp_1857.npz"), **out)


def layouts() -> None:
    cap = int(25.0 * 2**20)
    buckets, current, used = [], [], 0
    for name, shape in reversed(GPT2_SMALL):
        nbytes = _numel(shape) * 4
        if current and used + nbytes > cap:
            buckets.append(current)
            current, used = [], 0
        current.append([name, sum(c[2] for c in current), _numel(shape)])
        used += nbytes
    buckets.append(current)
    llama_total = sum(_numel(s) for _, s in LLAMA3_8B)
    data = {
        "gpt2_small_buckets_25mib": buckets,
        "gpt2_small_total": sum(_numel(s) for _, s in GPT2_SMALL),
        "mlp_1857": {str(w): [-(-1857 // w), -(-1857 // w) * w - 1857] for w in (1, 2, 3, 4, 8)},
        "llama3_8b": {"tensors": len(LLAMA3_8B), "total": llama_total,
                      "shards": {str(w): [-(-llama_total // w), -(-llama_total // w) * w - llama_total]
                                 for w in (2, 3, 4, 8)}},
        "llama3_70b": {"total": LLAMA3_70B_TOTAL, "w8_shard": LLAMA3_70B_TOTAL // 8},
        "reshard_12_4_to_3": [[[0, 3], [3, 1]], [[4, 2], [6, 2]], [[8, 1], [9, 3]]],
    }
    with open(os.path.join(HERE, "layouts.json"), "w", encoding="utf-8") as f:
        json.dump(data, f, indent=1)


if __name__ == "__main__":
    torch.set_num_threads(1)
    adamw_llama_shard()
    fsdp_mlp()
    layouts()
    print("golden vectors written to", HERE)
