"""Seeded random FSDP configurations through the whole flat-parameter path (GPU).

Each case draws a parameter list (odd sizes, empty tensors and multiples of 256 mixed,
so plans take both the aligned and the general copy kernel), a group size, parameter
and gradient dtypes and a reduce dtype, then checks every rank bitwise against the
oracle: the packed shard (``parallel/fsdp.py:434-454``), the gathered tensors
(``:912-925``), the gradient local share (``:704-781``) and a two-micro-batch
``no_sync`` reduction (``:733-749``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import FlatParamHandle, FSDPConfig, GroupHandle, MixedPrecisionConfig

pytestmark = pytest.mark.gpu

_NAMES = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}


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


@pytest.mark.parametrize("case", range(120))
def test_random_fsdp_configurations(device, case):
    rng = np.random.default_rng(1000 + case)
    shapes = _shapes(rng)
    group = int(rng.integers(1, 10))
    param_dtype = [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
    grad_dtype = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    reduce = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
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
