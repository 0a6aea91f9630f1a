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


def test_bucket_size_is_never_numerical(device):
    """``tests/distributed/test_ddp.py:314-358``: the bucket cap moves bucket boundaries
    only.  Caps that give one parameter per bucket, a few buckets or a single bucket
    yield the same averaged gradients bitwise, and the statistics count every byte."""
    named = [(f"p{i}", torch.nn.Parameter(torch.empty(n, device=device)))
             for i, n in enumerate([5, 1031, 64, 7, 4096, 3, 65536, 300])]
    gen = torch.Generator(device=device).manual_seed(9)
    grads = [torch.randn(p.shape, device=device, generator=gen) for _, p in named]
    group = GroupHandle.local_view("data_parallel", 3, 0)
    results, counts = [], []
    for cap_mb in (1e-6, 0.01, 25.0):
        for (_, p), g in zip(named, grads):
            p.grad = g.clone()
        ddp = BucketedGradients(named, group, DDPConfig(bucket_cap_mb=cap_mb))
        ddp.synchronize()
        counts.append(len(ddp.buckets))
        results.append([p.grad.detach().cpu().view(torch.int32).clone() for _, p in named])
        assert ddp.statistics.bytes_reduced == 4 * sum(p.numel() for _, p in named)
        assert ddp.statistics.buckets_reduced == len(ddp.buckets)
    assert counts[0] == len(named) and counts[-1] == 1 and counts[0] > counts[1] > counts[2]
    expect = [(g.detach().cpu().numpy() / np.float32(3)).astype(np.float32) for g in grads]
    for packed in results:
        for got, want in zip(packed, expect):
            assert np.array_equal(got.numpy(), want.view(np.int32))


def test_non_contiguous_gradients_are_packed(device):
    """A non-contiguous gradient is packed from a dense copy that stays alive until the
    pack has run; the averaged values are bitwise numpy's."""
    shapes = [(33, 17), (5,), (8, 64), (129, 3), (7,)]
    named = [(f"w{i}", torch.nn.Parameter(torch.empty(s, device=device))) for i, s in enumerate(shapes)]
    gen = torch.Generator(device=device).manual_seed(13)
    expect = {}
    for name, p in named:
        if p.dim() == 2:
            p.grad = torch.randn(tuple(reversed(p.shape)), device=device, generator=gen).t()
            assert not p.grad.is_contiguous()
        else:
            p.grad = torch.randn(p.shape, device=device, generator=gen)
        expect[name] = (p.grad.detach().cpu().contiguous().numpy() / np.float32(2)).astype(np.float32)
    ddp = BucketedGradients(named, GroupHandle.local_view("data_parallel", 2, 0), DDPConfig(bucket_cap_mb=25.0))
    ddp.synchronize()
    for name, p in named:
        assert p.grad.is_contiguous()
        assert np.array_equal(p.grad.detach().cpu().numpy().view(np.int32), expect[name].view(np.int32)), name


def test_no_sync_accumulates_then_packs_the_sum(device):
    """``ddp.py:702-733``: inside ``no_sync`` the buckets stay untouched while the
    micro-batches' gradients accumulate in ``param.grad`` (as autograd adds them); the
    first synchronisation outside packs the averaged sum, bitwise numpy's."""
    named = [(f"w{i}", torch.nn.Parameter(torch.empty(n, device=device))) for i, n in enumerate([300, 7, 4096])]
    gen = torch.Generator(device=device).manual_seed(17)
    micro = [[torch.randn(p.shape, device=device, generator=gen) for _, p in named] for _ in range(3)]
    ddp = BucketedGradients(named, GroupHandle.local_view("data_parallel", 4, 0), DDPConfig())
    for (_, p), g in zip(named, micro[0]):
        p.grad = g.clone()
    with ddp.no_sync():
        ddp.synchronize()
        for (_, p), g in zip(named, micro[1]):
            p.grad.add_(g)
        ddp.pack()
    assert ddp.statistics.steps == 0 and not any(b.is_allocated for b in ddp.buckets)
    for (_, p), g in zip(named, micro[2]):
        p.grad.add_(g)
    ddp.synchronize()
    assert ddp.statistics.steps == 1
    for i, (name, p) in enumerate(named):
        total = micro[0][i].cpu().numpy() + micro[1][i].cpu().numpy()
        total = (total + micro[2][i].cpu().numpy()).astype(np.float32)
        expect = (total / np.float32(4)).astype(np.float32)
        assert np.array_equal(p.grad.detach().cpu().numpy().view(np.int32), expect.view(np.int32)), name


def test_pack_with_ieee_specials(device):
    """IEEE specials through the bucket pack and its AVG divide (W=3, not a power of two,
    so a true division): ±inf, NaN, -0.0, the largest finite value and denormals, in an
    fp32 and a bf16 bucket; every non-NaN element bitwise numpy's ``g / 3`` rounded to
    the bucket dtype, NaNs in the same places."""
    shapes = [(4099,), (33, 17)]
    named = [(f"w{i}", torch.nn.Parameter(torch.empty(s, device=device, dtype=dt)))
             for i, (s, dt) in enumerate(zip(shapes, (torch.float32, torch.bfloat16)))]
    gen = torch.Generator(device=device).manual_seed(19)
    for _, p in named:
        g = torch.randn(p.shape, device=device, generator=gen).reshape(-1)
        g[:7] = torch.tensor([float("inf"), -float("inf"), float("nan"), -0.0,
                              torch.finfo(p.dtype).max, 1e-40, -1e-45], device=device)
        p.grad = g.to(p.dtype).reshape(p.shape)
    expect = {}
    for name, p in named:
        wide = p.grad.detach().float().cpu().numpy().reshape(-1)
        expect[name] = torch.from_numpy((wide / np.float32(3)).astype(np.float32)).to(p.dtype)
    ddp = BucketedGradients(named, GroupHandle.local_view("data_parallel", 3, 0), DDPConfig())
    ddp.synchronize()
    for name, p in named:
        got = p.grad.detach().cpu().reshape(-1)
        want = expect[name]
        nan = torch.isnan(want)
        assert torch.equal(torch.isnan(got), nan), name
        bits = torch.int16 if p.dtype == torch.bfloat16 else torch.int32
        assert torch.equal(got[~nan].view(bits), want[~nan].view(bits)), name


@pytest.mark.parametrize("world", [8, 3])
def test_repeated_packs_follow_gradient_changes(device, world):
    """A full pack over the same dense gradients reuses the last full pack's launches;
    each change the rows depend on (a gradient in another tensor, a non-contiguous
    gradient, a missing one) is packed afresh, and every pack equals ``grad / W``."""
    shapes = [(7, 5), (13,), (4, 4, 3), (1,), (33,)]
    named = [(f"p{i}", torch.nn.Parameter(torch.empty(s, device=device))) for i, s in enumerate(shapes)]
    gen = torch.Generator(device=device).manual_seed(world)

    def fresh(shape):
        return torch.randn(shape, device=device, generator=gen)

    for _, p in named:
        p.grad = fresh(p.shape)
    ddp = BucketedGradients(named, GroupHandle.local_view("dp", world, 0),
                            DDPConfig(bucket_cap_mb=0.0001, find_unused_parameters=True))
    assert len(ddp.buckets) > 1

    def packed_equals_grads():
        ddp.pack()
        for bucket in ddp.buckets:
            buf = bucket.buffer.cpu().numpy()
            for param, off, numel in zip(bucket.parameters, bucket.layout.offsets, bucket.layout.numels):
                g = param.grad
                expect = (np.zeros(numel, np.float32) if g is None
                          else (g.detach().cpu().numpy().reshape(-1) / np.float32(world)).astype(np.float32))
                assert np.array_equal(buf[off : off + numel].view(np.int32), expect.view(np.int32))

    packed_equals_grads()
    memo = ddp._pack_memo
    assert memo is not None
    for _, p in named:  # new values in the same tensors: the remembered launches
        p.grad.copy_(fresh(p.shape))
    packed_equals_grads()
    assert ddp._pack_memo is memo
    named[1][1].grad = fresh(shapes[1])  # another tensor
    packed_equals_grads()
    assert ddp._pack_memo is not memo and ddp._pack_memo is not None
    named[0][1].grad = fresh((5, 7)).t()  # non-contiguous: packed through a dense copy, not remembered
    packed_equals_grads()
    assert ddp._pack_memo is None
    named[0][1].grad = fresh(shapes[0])
    named[2][1].grad = None  # unused: zeros, not remembered
    packed_equals_grads()
    assert ddp._pack_memo is None and ddp.statistics.unused_parameters == ("p2",)
    named[2][1].grad = fresh(shapes[2])
    packed_equals_grads()
    assert ddp._pack_memo is not None and ddp.statistics.unused_parameters == ()
    for _, p in named:
        p.grad.mul_(3.0)
    packed_equals_grads()
    assert ddp.statistics.buckets_reduced == 7 * len(ddp.buckets)  # seven full packs
