"""GPU parity of the 2-byte master paths and of every dtype conversion of the reshard.

* AdamW and SGD on bfloat16 / float16 master shards (the reference's flat shards when
  mixed precision is off and the model is bf16 or fp16: ``parallel/fsdp.py:379-384``,
  ``optim/sharded_optimizer.py:111-126``): parameters and state bitwise equal to the
  oracle, and to ``torch.optim.AdamW`` / ``torch.optim.SGD(foreach=False)`` stepping the
  same tensors on the CPU after the reference's clip (fp64 norm, Python-double
  coefficient, ``grad.mul_`` in the gradient's dtype), NaN compared as NaN.
* An FSDP unit of bf16 parameters with mixed precision off: the shard, the local share
  reduced and stored in bf16, and the optimizer step, against the oracle pipeline.
* ``read_tensor_range`` into and out of float64 and between bfloat16 and float16
  (``checkpoint/reshard.py:290``, ``.to(out.dtype)``): bitwise equal to torch's CPU
  ``Tensor.to`` on the same values, IEEE specials included.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import (
    DeviceShardCache,
    FlatParamHandle,
    FSDPConfig,
    GroupHandle,
    MixedPrecisionConfig,
    OptimizerConfig,
    ShardedOptimizer,
    ShardRange,
    ShardRecord,
    TensorRecord,
    read_tensor_range,
    shard_filename,
)

pytestmark = pytest.mark.gpu

_NAMES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.element_size() == 2:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.element_size() == 4:
        return t.view(torch.int32).numpy()
    return t.view(torch.int64).numpy()


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equal, a NaN matching any NaN."""
    a, b = a.detach().cpu(), b.detach().cpu()
    nan = torch.isnan(a.float())
    if not torch.equal(nan, torch.isnan(b.float())):
        return False
    return bool(np.array_equal(_bits(a)[~nan.numpy()], _bits(b)[~nan.numpy()]))


def _reference_clip(params: list[torch.nn.Parameter], max_norm: float) -> float:
    """optim/sharded_optimizer.py:310-338 on CPU tensors: fp64 norm, Python coefficient,
    grad.mul_ in the gradient's dtype."""
    norm = float(sum(p.grad.detach().to(torch.float64).pow(2).sum() for p in params) ** 0.5)
    coef = max_norm / (norm + 1e-6)
    if coef < 1.0:
        for p in params:
            p.grad.detach().mul_(coef)
    return norm


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", ["adamw", "sgd"])
def test_lowp_master_steps_match_torch_and_the_oracle(device, dtype, name):
    sizes = [1, 7, 511, 512, 513, 4097, 100_003]  # tails and whole 512-element tiles
    gen = torch.Generator().manual_seed(9)
    host = [torch.nn.Parameter((torch.randn(n, generator=gen) * 0.05).to(dtype)) for n in sizes]
    params = [torch.nn.Parameter(p.detach().to(device)) for p in host]
    if name == "adamw":
        config = OptimizerConfig(learning_rate=1e-3, betas=(0.9, 0.95), eps=1e-4, weight_decay=0.1)
        ref = torch.optim.AdamW(host, lr=1e-3, betas=(0.9, 0.95), eps=1e-4, weight_decay=0.1, foreach=False)
    else:
        config = OptimizerConfig(name="sgd", learning_rate=0.05, momentum=0.9, weight_decay=0.01)
        ref = torch.optim.SGD(host, lr=0.05, momentum=0.9, weight_decay=0.01, foreach=False)
    opt = ShardedOptimizer(params, config, norm_group=GroupHandle.trivial(), device=device)
    dt = _NAMES[dtype]
    P = [oracle.to_bits(p.detach().float().numpy(), dt) for p in host]
    S1 = [np.zeros(n, np.uint16) for n in sizes]
    S2 = [np.zeros(n, np.uint16) for n in sizes]
    for step in range(1, 5):
        grads = [(torch.randn(n, generator=gen) * 0.3).to(dtype) for n in sizes]  # norm ~ 30: clipped
        for h, p, g in zip(host, params, grads):
            h.grad = g.clone()
            p.grad = g.to(device)
        norm = float(opt.clip_grad_norm(1.0))
        opt.step()
        # torch's CPU kernels end every thread's range with a scalar remainder loop; with
        # one thread, as the reference's harness runs (tests/conftest.py:62-63), that loop
        # covers only each tensor's last n mod V elements
        threads = torch.get_num_threads()
        torch.set_num_threads(1)
        try:
            ref_norm = _reference_clip(host, 1.0)
            ref.step()
        finally:
            torch.set_num_threads(threads)
        assert abs(norm - ref_norm) <= 1e-12 * ref_norm
        mul = oracle.clip_multiplier(norm, 1.0)
        # the two norms round to the same fp32 multiplier, so torch's steps are comparable bitwise
        assert mul == oracle.clip_multiplier(ref_norm, 1.0) < 1.0
        for k, g in enumerate(grads):
            gb = _bits(g)
            if name == "adamw":
                sc = oracle.adamw_scalars(lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-4, weight_decay=0.1, step=float(step))
                oracle.adamw_step(P[k], gb, S1[k], S2[k], sc, grad_mul=mul, dtype=dt)
            else:
                oracle.sgd_step(P[k], gb, S1[k], lr=0.05, momentum=0.9, weight_decay=0.01, first=step == 1,
                                grad_mul=mul, dtype=dt)
        for k, (h, p) in enumerate(zip(host, params)):
            context = (name, dt, step, sizes[k])
            # torch's own optimizer on the CPU: every element for AdamW; for SGD the
            # elements of torch's vectorised body (its vector width divides 64), since its
            # scalar remainder loop rounds each alpha product to the dtype first (the
            # oracle's `remainder` form; the kernels follow the body everywhere)
            body = sizes[k] if name == "adamw" else sizes[k] - sizes[k] % 64
            state, ref_state = opt.inner.state[p], ref.state[h]
            first = "exp_avg" if name == "adamw" else "momentum_buffer"
            assert np.array_equal(_bits(p), P[k]), context
            assert np.array_equal(_bits(state[first]), S1[k]), context
            assert _same(p[:body], h[:body]), context
            assert _same(state[first][:body], ref_state[first][:body]), context
            assert _same(p.grad, h.grad), context  # the clipped gradient written back in place
            if name == "adamw":
                assert np.array_equal(_bits(state["exp_avg_sq"]), S2[k]), context
                assert _same(state["exp_avg_sq"], ref_state["exp_avg_sq"]), context
        opt.zero_grad(set_to_none=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_bf16_fsdp_unit_without_mixed_precision(device, dtype):
    """Mixed precision off and bf16 / fp16 parameters: the master, compute and reduce
    dtypes are all the parameters' (``fsdp.py:379-392``).  Each rank's shard packs
    bitwise, its gradient shard is the AVG reduce-scatter in that dtype (rank order)
    stored in that dtype with the padding zero, and the AdamW step on it matches the
    oracle bitwise."""
    dt = _NAMES[dtype]
    group = 4
    shapes = [(25, 14), (25,), (25, 25), (25,), (7, 25), (7,)]
    gen = torch.Generator(device=device).manual_seed(2)
    originals = [(torch.randn(s, device=device, generator=gen) * 0.1).to(dtype) for s in shapes]
    total = sum(t.numel() for t in originals)
    flat_host = torch.cat([t.reshape(-1).cpu() for t in originals])
    handles = []
    for rank in range(group):
        named = [(f"p{i}", torch.nn.Parameter(t.clone())) for i, t in enumerate(originals)]
        handles.append(FlatParamHandle(named, None, GroupHandle.local_view("shard", group, rank), FSDPConfig(),
                                       MixedPrecisionConfig(enabled=False), device))
    shard = handles[0].shard_numel
    assert shard == -(-total // group) and handles[0].flat_param.dtype == dtype
    padded = torch.zeros(shard * group, dtype=dtype)
    padded[:total] = flat_host
    full_grads = [(torch.randn(shard * group, device=device, generator=gen) * 1e-2).to(dtype) for _ in range(group)]
    for g in full_grads:
        g[total:] = 0.0
    host_grads = [g.float().cpu().numpy() for g in full_grads]
    for rank, handle in enumerate(handles):
        assert torch.equal(handle.flat_param.detach().cpu(), padded[rank * shard : (rank + 1) * shard])
        out = handle.reduce_scatter_gradient(full_grads[rank], peer_grads=full_grads)
        assert out.dtype == dtype
        valid = max(0, min(shard, total - rank * shard))
        expect = oracle.to_bits(oracle.local_share(host_grads, rank, shard, valid, float(group), dt), dt)
        assert np.array_equal(_bits(out), expect), rank
        param = handle.flat_param
        param.grad = out
        opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=1e-3, betas=(0.9, 0.999), eps=1e-4,
                                                        weight_decay=0.01),
                               norm_group=GroupHandle.local_view("world", group, rank), device=device)
        P = _bits(param).copy()
        opt.clip_grad_norm(0.0)  # norm only (from the local share's partials)
        opt.step()
        sc = oracle.adamw_scalars(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-4, weight_decay=0.01, step=1.0)
        oracle.adamw_step(P, expect, np.zeros(shard, np.uint16), np.zeros(shard, np.uint16), sc, dtype=dt)
        assert np.array_equal(_bits(param), P), rank


_CONVERT = [torch.float64, torch.float32, torch.bfloat16, torch.float16]


@pytest.mark.parametrize("src", _CONVERT)
@pytest.mark.parametrize("dst", _CONVERT)
def test_read_tensor_range_converts_like_tensor_to(device, src, dst):
    if src == dst:
        pytest.skip("same-dtype reads are bit copies (test_gpu_reshard)")
    gen = torch.Generator().manual_seed(4)
    n = 50_001
    exps = torch.rand(n, generator=gen, dtype=torch.float64) * 80 - 40
    values = torch.randn(n, generator=gen, dtype=torch.float64) * torch.pow(2.0, exps)
    specials = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 65504.0, 65520.0, 1e-8,
                             6e-8, 3e38, 3.5e38, 1e-40, 1e-300, 1e300, 2.0**-149, 1.0 + 2.0**-30], dtype=torch.float64)
    values[: specials.numel()] = specials
    stored = values.to(src)
    # two writer shards, read over a range that straddles them at an odd offset
    cut = 20_011
    rec = TensorRecord(key="w", name="w", global_shape=(n,), dtype=str(src).replace("torch.", ""))
    cache = DeviceShardCache()
    for rank, (lo, hi) in enumerate([(0, cut), (cut, n)]):
        key = f"model::w@{lo}"
        rec.shards.append(ShardRecord(rank=rank, file=shard_filename(rank), offset=lo, length=hi - lo, key=key))
        cache.add(shard_filename(rank), key, stored[lo:hi].to(device))
    rec.validate()
    wanted = ShardRange(3, n - 10)
    got = read_tensor_range(rec, wanted, cache, dtype=dst)
    assert got.dtype == dst and got.numel() == wanted.length
    expect = stored[3 : n - 7].to(dst)
    assert _same(got, expect), (src, dst)
