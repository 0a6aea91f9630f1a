"""The oracle and the host logic against the committed golden vectors (no GPU).

Golden vectors come from ``tests/golden/make_golden.py``: torch.optim.AdamW on the CPU
(the reference's optimizer) driven by the reference's clip sequence, and layout tables
from the reference's rules.  The oracle reproduces m and v bitwise (they do not depend
on the square root) and p within ``|a - b| <= 1e-6 * max(|b|, lr)`` (torch's CPU sqrt
on large tensors is not correctly rounded; the oracle's is).
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

import oracle
from hybrid_training_amd import build_buckets, concat_shard_sizes

from .model_shapes import GPT2_SMALL, LLAMA3_8B

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RTOL = 1e-6


def _rel(a, b, floor):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), floor)))


def test_oracle_reproduces_the_clipped_adamw_trajectory():
    g = np.load(os.path.join(GOLDEN, "adamw_llama_shard_4096.npz"))
    lr, b1, b2, eps, wd, max_norm = (float(x) for x in g["hyper"])
    p = g["p0"].copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for k in range(g["grads"].shape[0]):
        grad = g["grads"][k]
        norm = float(np.sqrt(oracle.sqnorm(grad)))
        assert abs(norm - g["norms"][k]) <= 1e-12 * g["norms"][k]
        mul = oracle.clip_multiplier(norm, max_norm)
        assert np.float32(mul) == np.float32(g["coefs"][k])
        sc = oracle.adamw_scalars(lr=lr, beta1=b1, beta2=b2, eps=eps, weight_decay=wd, step=float(k + 1))
        oracle.adamw_step(p, grad, m, v, sc, grad_mul=mul)
    assert np.array_equal(m, g["m"]) and np.array_equal(v, g["v"])
    assert _rel(p, g["p"], lr) <= RTOL


def test_oracle_reproduces_the_fsdp_mlp_shards():
    g = np.load(os.path.join(GOLDEN, "fsdp_mlp_1857.npz"))
    for world in (2, 4):
        shards = g[f"w{world}_initial"].copy()
        m = np.zeros_like(shards)
        v = np.zeros_like(shards)
        for step in range(5):
            sc = oracle.adamw_scalars(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
                                      step=float(step + 1))
            for r in range(world):
                oracle.adamw_step(shards[r], g[f"w{world}_grads"][step, r], m[r], v[r], sc)
            assert _rel(shards, g[f"w{world}_shards"][step], 1e-3) <= RTOL
        total = 1857
        flat = np.concatenate(list(shards))
        assert np.all(flat[total:] == 0.0)


def test_layout_tables():
    with open(os.path.join(GOLDEN, "layouts.json"), encoding="utf-8") as f:
        data = json.load(f)
    named = [(n, torch.nn.Parameter(torch.empty(s, device="meta"))) for n, s in GPT2_SMALL]
    buckets = build_buckets(named, 25.0)
    table = [[[n, o, k] for n, o, k in zip(b.layout.parameter_names, b.layout.offsets, b.layout.numels)]
             for b in buckets]
    assert table == data["gpt2_small_buckets_25mib"]
    for w, (shard, pad) in data["mlp_1857"].items():
        assert concat_shard_sizes(1857, int(w)) == (shard * int(w), shard) and shard * int(w) - 1857 == pad
    total = sum(int(torch.Size(s).numel()) for _, s in LLAMA3_8B)
    assert total == data["llama3_8b"]["total"]
    for w, (shard, pad) in data["llama3_8b"]["shards"].items():
        assert concat_shard_sizes(total, int(w)) == (shard * int(w), shard)
