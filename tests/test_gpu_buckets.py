"""GPU parity of DDP bucket packing with the AVG pre-divide, at GPT-2-small size.

124,439,808 fp32 gradients ~ N(0, 1e-3) in 17 buckets of <= 25 MiB: after ``pack``
each bucket slice must equal the gradient divided by W in fp32, bitwise (numpy's
float32 division is IEEE, as torch's ``div_`` is); after ``bind_gradients`` every
``param.grad`` is a view of its bucket.  W=8 (a power of two) and W=3 both run.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from hybrid_training_amd import BucketedGradients, DDPConfig, GroupHandle, ShardingError

from .model_shapes import GPT2_SMALL

pytestmark = pytest.mark.gpu


def _gpt2_params(device):
    return [(n, torch.nn.Parameter(torch.empty(s, device=device))) for n, s in GPT2_SMALL]


@pytest.mark.parametrize("world", [8, 3, 1])
def test_gpt2_small_pack_and_average(device, world):
    named = _gpt2_params(device)
    gen = torch.Generator(device=device).manual_seed(world)
    for _, p in named:
        p.grad = torch.randn(p.shape, device=device, generator=gen) * 1e-3
    grads = {n: p.grad.detach().cpu().numpy().reshape(-1) for n, p in named}
    group = GroupHandle.local_view("data_parallel", world, 0) if world > 1 else GroupHandle.trivial()
    ddp = BucketedGradients(named, group, DDPConfig(bucket_cap_mb=25.0))
    assert len(ddp.buckets) == 17
    ddp.synchronize()
    divisor = np.float32(world)
    for bucket in ddp.buckets:
        buf = bucket.buffer.cpu().numpy()
        for name, off, numel in zip(bucket.layout.parameter_names, bucket.layout.offsets, bucket.layout.numels):
            expect = grads[name] if world == 1 else (grads[name] / divisor).astype(np.float32)
            assert np.array_equal(buf[off : off + numel].view(np.int32), expect.view(np.int32)), name
    # gradient-as-bucket-view: no copy back
    for bucket in ddp.buckets:
        for position, param in enumerate(bucket.parameters):
            assert param.grad.data_ptr() == bucket.buffer.data_ptr() + bucket.layout.offsets[position] * 4
            assert param.grad.shape == param.shape
    assert ddp.statistics.steps == 1 and ddp.statistics.buckets_reduced == 17
    # A second synchronisation with the gradients already living in the buckets.
    for _, p in named:
        p.grad.mul_(2.0)
    ddp.synchronize()
    name, param = named[5]
    expect = grads[name] * np.float32(2.0) if world == 1 else (
        (grads[name] / divisor).astype(np.float32) * np.float32(2.0) / divisor).astype(np.float32)
    assert np.array_equal(param.grad.detach().cpu().numpy().reshape(-1), expect.astype(np.float32))


def test_unused_parameters(device):
    named = [("a", torch.nn.Parameter(torch.ones(5, device=device))),
             ("b", torch.nn.Parameter(torch.ones(3, device=device)))]
    named[0][1].grad = torch.full((5,), 4.0, device=device)
    ddp = BucketedGradients(named, GroupHandle.local_view("dp", 2, 0), DDPConfig())
    with pytest.raises(ShardingError, match="received no gradient"):
        ddp.synchronize()
    ddp = BucketedGradients(named, GroupHandle.local_view("dp", 2, 0), DDPConfig(find_unused_parameters=True))
    ddp.synchronize()
    assert torch.equal(named[1][1].grad.cpu(), torch.zeros(3))
    assert torch.equal(named[0][1].grad.cpu(), torch.full((5,), 2.0))
    assert ddp.statistics.unused_parameters == ("b",)


def test_parameterless_module_rejected(device):
    with pytest.raises(ShardingError, match="no trainable parameters"):
        BucketedGradients([], GroupHandle.trivial(), DDPConfig())


def test_bucket_by_bucket_pack_matches_one_launch(device):
    """Packing the buckets one at a time, in the order a backward pass completes them
    (reverse registration order, bucket 0 first), gives the same bits as one launch."""
    named = _gpt2_params(device)
    gen = torch.Generator(device=device).manual_seed(11)
    grads = [torch.randn(p.shape, device=device, generator=gen) * 1e-3 for _, p in named]
    group = GroupHandle.local_view("data_parallel", 8, 0)
    results = []
    for per_bucket in (False, True):
        for (_, p), g in zip(named, grads):
            p.grad = g.clone()
        ddp = BucketedGradients(named, group, DDPConfig(bucket_cap_mb=25.0))
        if per_bucket:
            for index in range(len(ddp.buckets)):
                ddp.pack([index])
        else:
            ddp.pack()
        results.append([b.buffer.detach().cpu().clone() for b in ddp.buckets])
        assert ddp.statistics.buckets_reduced == 17
    for a, b in zip(*results):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    with pytest.raises(ShardingError, match="distinct and in range"):
        ddp.pack([17])
    with pytest.raises(ShardingError, match="distinct and in range"):
        ddp.pack([3, 3])
