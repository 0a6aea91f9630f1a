"""Host-only behaviour: error messages, configuration validation, the scaler state
machine and the oracle's local-share and no_sync restatements (no GPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import (
    DDPConfig,
    FSDPConfig,
    GradScalerConfig,
    GroupHandle,
    MixedPrecisionConfig,
    OptimizerConfig,
    format_error,
)
from hybrid_training_amd.errors import ConfigurationError, UnsupportedFeatureError
from hybrid_training_amd.grad_scaler import GradScaler, GradScalerState


def test_format_error_matches_the_reference_example():
    msg = format_error(
        "topology.validate",
        "parallel sizes do not factor the world size",
        rank=3, world_size=8, expected=8, observed=6,
        resolution="set dp*shard*seq*tensor == world_size",
    )
    assert msg == (
        "[rank 3/8] topology.validate: parallel sizes do not factor the world size; "
        "expected 8, observed 6. Fix: set dp*shard*seq*tensor == world_size"
    )
    assert format_error("a.b", "bad") == "a.b: bad"
    assert format_error("a.b", "bad", rank=1) == "[rank 1] a.b: bad"


def test_config_validation():
    with pytest.raises(ConfigurationError, match="bucket_cap_mb must be positive"):
        DDPConfig(bucket_cap_mb=0)
    with pytest.raises(ConfigurationError, match="use_padding=False is not supported"):
        FSDPConfig(use_padding=False)
    with pytest.raises(ConfigurationError, match="betas must be two values"):
        OptimizerConfig(betas=(0.9, 1.0))
    with pytest.raises(ConfigurationError, match="unknown optimizer"):
        OptimizerConfig(name="lamb")
    with pytest.raises(ConfigurationError, match="backoff_factor"):
        GradScalerConfig(backoff_factor=1.5)
    with pytest.raises(ConfigurationError, match="only meaningful for float16"):
        MixedPrecisionConfig(enabled=True, param_dtype="bfloat16", scaler=GradScalerConfig(enabled=True))
    assert OptimizerConfig().weight_decay == 0.0 and OptimizerConfig().eps == 1e-8


def test_scaler_state_machine():
    cfg = GradScalerConfig(enabled=True, init_scale=65536.0, growth_interval=3, max_scale=2.0**17)
    scaler = GradScaler(cfg, GroupHandle.trivial(), device="cpu")
    assert scaler.scale_value == 65536.0
    assert scaler.update(found_non_finite=True) == 32768.0
    assert scaler.state.growth_tracker == 0
    for _ in range(2):
        assert scaler.update(found_non_finite=False) == 32768.0
    assert scaler.update(found_non_finite=False) == 65536.0
    for _ in range(6):
        scaler.update(found_non_finite=False)
    assert scaler.scale_value == 2.0**17  # capped at max_scale
    low = GradScaler(GradScalerConfig(enabled=True, init_scale=1.0), GroupHandle.trivial(), device="cpu")
    assert low.update(found_non_finite=True) == 1.0  # floor at 1
    state = scaler.state_dict()
    again = GradScaler(cfg, GroupHandle.trivial(), device="cpu")
    again.load_state_dict(state)
    assert again.state == GradScalerState.from_dict(state)
    disabled = GradScaler(GradScalerConfig(), GroupHandle.trivial(), device="cpu")
    assert disabled.scale_value == 1.0 and disabled.update() == 1.0


def test_group_handles():
    g = GroupHandle.trivial()
    assert g.size == 1 and g.is_trivial and g.process_group is None
    v = GroupHandle.local_view("shard", 4, 2)
    assert v.size == 4 and v.local_rank == 2 and not v.is_trivial


def test_real_process_groups_are_refused():
    import torch

    from hybrid_training_amd import ShardedOptimizer

    group = GroupHandle(name="world", ranks=(0, 1), local_rank=0, global_rank=0, process_group=object())
    with pytest.raises(UnsupportedFeatureError, match="no collectives"):
        ShardedOptimizer([torch.nn.Parameter(torch.zeros(2))], OptimizerConfig(), norm_group=group,
                         device=torch.device("cpu"))


def test_oracle_local_share_against_torch_avg():
    """The reference's AVG local share with torch's own ops.

    Each rank's padded gradient is divided by G with ``Tensor.div`` (IEEE division,
    ``distributed/collectives.py:593-594``), the reduce-scatter sums the divided
    buffers, and the padding tail is zeroed (``parallel/fsdp.py:771-781``).  For G <= 2
    the sum does not depend on its order (IEEE addition commutes), so torch pins the
    result bitwise; it is formed here in reverse rank order to show that.  For G > 2
    the rank order is the fixed order the oracle and the kernel share.
    """
    import functools

    import torch

    gen = torch.Generator().manual_seed(0)
    for group, shard, pad in ((1, 7, 2), (2, 5, 1), (3, 5, 2), (4, 6, 3)):
        total = group * shard - pad
        grads = [torch.randn(group * shard, generator=gen) for _ in range(group)]
        divided = [g.div(group) for g in grads]
        if group <= 2:
            summed = functools.reduce(torch.add, reversed(divided))
        else:
            summed = functools.reduce(torch.add, divided)
        summed[total:] = 0.0
        host = [g.numpy() for g in grads]
        for rank in range(group):
            valid = max(0, min(shard, total - rank * shard))
            got = oracle.local_share(host, rank, shard, valid, float(group))
            assert np.array_equal(got, summed[rank * shard : (rank + 1) * shard].numpy()), (group, rank)
            assert np.all(got[valid:] == 0.0)


def _torch_no_sync(micro, reduce=torch.float32):
    """The reference's own op sequence on CPU (``parallel/fsdp.py:733-749``)."""
    accumulator = None
    for g in micro[:-1]:
        grad = g.to(reduce).contiguous()
        if accumulator is None:
            accumulator = grad.clone()
        else:
            accumulator.add_(grad)
    grad = micro[-1].to(reduce).contiguous()
    return grad if accumulator is None else grad + accumulator


_REDUCE_NAMES = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}


@pytest.mark.parametrize("reduce", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("micro", [1, 2, 3, 5])
def test_oracle_no_sync_accumulate_against_torch(reduce, dtype, micro):
    """Bitwise against torch on CPU, with signed zeros (a copy keeps -0.0 where adding
    to zeros would not), subnormal sums, overflow and random values."""
    gen = torch.Generator().manual_seed(micro)
    n = 4096
    grads = []
    for m in range(micro):
        g = (torch.randn(n, generator=gen) * 1e-2).to(dtype)
        g[:8] = -0.0                          # -0.0 in every micro-batch
        g[8] = 0.0 if m else -0.0             # -0.0 then +0.0: the sum is +0.0
        g[9] = torch.finfo(dtype).tiny / 4    # subnormal (fp32, fp16) or a tiny normal sum
        g[10] = torch.finfo(dtype).max        # overflows in the sum or in the cast to a narrower dtype
        g[11] = -torch.finfo(dtype).max
        grads.append(g)
    expect = _torch_no_sync(grads, reduce).to(torch.float32)
    got = oracle.no_sync_accumulate([g.float().numpy() for g in grads], _REDUCE_NAMES[reduce])
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), expect.numpy().view(np.uint32))
    if micro > 1:
        assert np.all(np.signbit(got[:8])) and not np.signbit(got[8])
        if reduce is torch.float32 and dtype == torch.float16:
            # The sum is formed in fp32, where micro * 65504 is exact; fp16 would overflow.
            assert got[10] == 65504.0 * micro and got[11] == -65504.0 * micro
        elif reduce is torch.bfloat16 and dtype == torch.float16:
            assert np.isfinite(got[10]) and got[10] > 0 and np.isfinite(got[11]) and got[11] < 0
        else:
            assert np.isinf(got[10]) and got[10] > 0 and np.isinf(got[11]) and got[11] < 0
        # Accumulating onto zeros instead of copying the first micro-batch loses the sign of -0.0.
        from_zeros = np.zeros(n, dtype=np.float32)
        with np.errstate(over="ignore"):
            for g in grads:
                from_zeros = np.add(from_zeros, g.float().numpy(), dtype=np.float32)
        assert not np.array_equal(from_zeros.view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_oracle_float64_local_share_against_torch_and_exact_mean(dtype):
    """``reduce_dtype="float64"``: torch's own ops (``Tensor.to(float64)``, ``div(G)``,
    the rank sum, ``Tensor.to(float32)``) pin the oracle bitwise for every G; for G a
    power of two the float64 sum of fp32-representable values of one scale is exact,
    so the result is also the exact rational mean rounded once to fp32."""
    import functools
    from fractions import Fraction

    gen = torch.Generator().manual_seed(3)
    for group, shard, pad in ((1, 9, 2), (2, 7, 1), (3, 8, 3), (4, 6, 0), (8, 5, 4)):
        total = group * shard - pad
        grads = [(torch.randn(group * shard, generator=gen) * 3.0).to(dtype) for _ in range(group)]
        wide = functools.reduce(torch.add, [g.to(torch.float64).div(group) for g in grads])
        wide[total:] = 0.0
        summed = wide.to(torch.float32)
        host = [g.float().numpy() for g in grads]
        for rank in range(group):
            valid = max(0, min(shard, total - rank * shard))
            got = oracle.local_share(host, rank, shard, valid, float(group), "float64")
            assert got.dtype == np.float32
            assert np.array_equal(got.view(np.uint32), summed[rank * shard:(rank + 1) * shard].numpy().view(np.uint32))
            # a float64 master keeps the float64 sum: torch's ops without the final cast
            kept = oracle.local_share(host, rank, shard, valid, float(group), "float64", out="float64")
            want = wide[rank * shard:(rank + 1) * shard].numpy()
            assert kept.dtype == np.float64 and np.array_equal(kept.view(np.uint64), want.view(np.uint64))
            if group & (group - 1) == 0:
                for i in range(valid):
                    exact = sum(Fraction(float(h[rank * shard + i])) for h in host) / group
                    assert Fraction(float(exact)) == exact  # representable in float64
                    assert got[i] == np.float32(float(exact))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("micro", [1, 2, 5])
def test_oracle_float64_no_sync_against_torch(dtype, micro):
    """The float64 accumulator: torch's op sequence pins the oracle bitwise, and for
    values of one scale the float64 sum is the exact sum."""
    from fractions import Fraction

    gen = torch.Generator().manual_seed(micro)
    grads = [(torch.randn(512, generator=gen) * 1e-2).to(dtype) for _ in range(micro)]
    grads[0][:4] = -0.0
    expect = _torch_no_sync(grads, torch.float64).numpy()
    got = oracle.no_sync_accumulate([g.float().numpy() for g in grads], "float64")
    assert got.dtype == np.float64
    assert np.array_equal(got.view(np.uint64), expect.view(np.uint64))
    for i in range(4, 512, 37):
        assert Fraction(float(got[i])) == sum(Fraction(float(g[i])) for g in grads)


@pytest.mark.parametrize("reduce", [torch.bfloat16, torch.float16])
def test_oracle_round_to_against_torch(reduce):
    """``round_to`` is torch's cast to the reduce dtype and back, on specials (ties,
    overflow, subnormals, signed zeros, infinities) and random values of every scale."""
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(1 << 16, generator=gen) * torch.logspace(-45, 38, 1 << 16, base=2.0)
    specials = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 65504.0, 65520.0, 65519.99,
                             3.3895314e38, 3.4028235e38, 1e-8, 5.9604645e-8, 2.9802322e-8,
                             1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11])
    x = torch.cat([specials, -specials, x])
    expect = x.to(reduce).to(torch.float32).numpy()
    got = oracle.round_to(x.numpy(), _REDUCE_NAMES[reduce])
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


@pytest.mark.parametrize("reduce", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_oracle_local_share_reduce_dtype_against_torch(reduce, dtype):
    """The reference's AVG local share in a 2-byte reduce dtype, with torch's own ops:
    ``Tensor.to(reduce)``, ``div(G)`` and the rank sum in that dtype, then the cast to
    the fp32 master and the padding zero.  Order-free for G <= 2, as in fp32."""
    import functools

    gen = torch.Generator().manual_seed(1)
    for group, shard, pad in ((1, 7, 2), (2, 64, 1), (3, 50, 2), (4, 66, 3)):
        total = group * shard - pad
        grads = [(torch.randn(group * shard, generator=gen) * 3.0).to(dtype) for _ in range(group)]
        divided = [g.to(reduce).div(group) for g in grads]
        summed = functools.reduce(torch.add, reversed(divided) if group <= 2 else divided).to(torch.float32)
        summed[total:] = 0.0
        host = [g.float().numpy() for g in grads]
        for rank in range(group):
            valid = max(0, min(shard, total - rank * shard))
            got = oracle.local_share(host, rank, shard, valid, float(group), _REDUCE_NAMES[reduce])
            expect = summed[rank * shard:(rank + 1) * shard].numpy()
            assert np.array_equal(got.view(np.uint32), expect.view(np.uint32)), (group, rank)
            if group > 1:
                # Reducing in fp32 instead gives different bits on some element.
                fp32 = oracle.local_share(host, rank, shard, valid, float(group))
                assert not np.array_equal(fp32.view(np.uint32), got.view(np.uint32))


def test_oracle_pack_matches_concatenation():
    rng = np.random.default_rng(1)
    tensors = [rng.standard_normal(s).astype(np.float32) for s in ((25, 14), (25,), (7, 25), (7,))]
    flat = np.concatenate([t.reshape(-1) for t in tensors])
    for group in (1, 2, 3, 4, 7):
        shard, padded, pad = oracle.even_shards(flat.size, group)
        pieces = [oracle.pack_shard(tensors, group, r) for r in range(group)]
        joined = np.concatenate(pieces)
        assert np.array_equal(joined[: flat.size], flat) and np.all(joined[flat.size :] == 0)
        back = oracle.unpack_full(joined, [t.shape for t in tensors])
        assert all(np.array_equal(a, b) for a, b in zip(back, tensors))


def test_every_oracle_function_says_how_it_is_pinned():
    """Each restatement in the oracle names the checks that pin it (known answers,
    library routines, closed forms, brute force); only the bit-view and loader helpers
    restate nothing."""
    helpers = {"library", "to_bits", "from_bits"}
    for name in oracle.__all__:
        if callable(getattr(oracle, name)) and name not in helpers:
            assert name in oracle.PINNED_BY, name
    assert set(oracle.PINNED_BY) <= set(oracle.__all__)


def test_norm_contribution_from_runs_matches_the_vector_form():
    from hybrid_training_amd import build_gradient_norm_contributions
    from hybrid_training_amd.flat_param import FlatParameter

    p = FlatParameter(torch.zeros(10), requires_grad=True)
    p.gradient_norm_scale_runs = [(0, 7, 2.0), (7, 3, 0.0)]
    (c,) = build_gradient_norm_contributions([p], world_size=4)
    assert c.scale is None and c.per_element and c.runs == [(0, 7, 0.5), (7, 3, 0.0)]
    assert torch.equal(c.scale_vector(), torch.tensor([0.5] * 7 + [0.0] * 3, dtype=torch.float64))
    # the reference's host vector, built lazily from the runs, gives the same runs
    assert torch.equal(p.gradient_norm_scale_vector, torch.tensor([2.0] * 7 + [0.0] * 3))
    q = torch.nn.Parameter(torch.zeros(10))
    q.gradient_norm_scale_vector = torch.tensor([2.0] * 7 + [0.0] * 3)
    (d,) = build_gradient_norm_contributions([q], world_size=4)
    assert d.runs == c.runs and torch.equal(d.scale_vector(), c.scale_vector())


def test_copy_plan_table_and_alignment_class():
    """The copy plan's records, chunk prefix sums and the aligned-kernel test (host only)."""
    from hybrid_training_amd import _native

    rows = [(4096, 8192, 600), (0, 65536, 256), (12288, 99328, 1)]
    flat, total = _native.plan_table(rows, 256)
    assert flat == [4096, 8192, 600, 0, 0, 65536, 256, 3, 12288, 99328, 1, 4]
    assert total == 5
    flat2, total2 = _native.plan_table(rows[:1], 256, scale=2)  # fp64 as dword pairs
    assert flat2 == [4096, 8192, 1200, 0] and total2 == 5
    f32, bf16, f16 = _native.DTYPE_F32, _native.DTYPE_BF16, _native.DTYPE_F16
    assert _native.plan_is_aligned(rows, f32, f32)
    assert not _native.plan_is_aligned([(4100, 8192, 4)], f32, f32)   # source off 16 B
    assert not _native.plan_is_aligned([(4096, 8200, 4)], f32, f32)   # destination off 16 B
    assert _native.plan_is_aligned([(4104, 8192, 4)], bf16, f32)      # 8-byte source units
    assert _native.plan_is_aligned([(4104, 8192, 4)], f16, f32)
    assert not _native.plan_is_aligned([(4100, 8192, 4)], bf16, f32)
    assert not _native.plan_is_aligned([(4104, 8192, 4)], f32, bf16)  # 16-byte source units
    assert _native.plan_is_aligned([(0, 8192, 4)], bf16, bf16)         # zero fill


def _mlp_23_32_32_1():
    torch.manual_seed(3)
    model = torch.nn.Sequential(torch.nn.Linear(23, 32), torch.nn.ReLU(), torch.nn.Linear(32, 32), torch.nn.ReLU(),
                                torch.nn.Linear(32, 1))
    return model, list(model.named_parameters())


def test_flat_param_handle_refuses_the_reference_failure_modes():
    """The reference's FSDP failure modes at the unit (``tests/distributed/test_fsdp.py:550-565``,
    ``parallel/fsdp.py:333-420``), refused before anything is packed: a unit mixing frozen
    and trainable parameters, a unit whose all-gather exceeds ``limit_all_gather_bytes``
    (1024 bytes against the MLP's 7,432 at W=2) and a unit with no parameters."""
    from hybrid_training_amd import (FlatParamHandle, FSDPConfig, GroupHandle, MixedPrecisionConfig, ShardingError,
                                     UnsupportedFeatureError)

    cpu = torch.device("cpu")
    group = GroupHandle.local_view("shard", 2, 0)
    model, named = _mlp_23_32_32_1()
    model[4].weight.requires_grad_(False)
    with pytest.raises(UnsupportedFeatureError, match="requires_grad"):
        FlatParamHandle(named, None, group, FSDPConfig(), MixedPrecisionConfig(), cpu)
    _, named = _mlp_23_32_32_1()
    with pytest.raises(ShardingError, match="limit_all_gather_bytes"):
        FlatParamHandle(named, None, group, FSDPConfig(limit_all_gather_bytes=1024), MixedPrecisionConfig(), cpu)
    with pytest.raises(ShardingError, match="at least one parameter"):
        FlatParamHandle([], None, group, FSDPConfig(), MixedPrecisionConfig(), cpu)
    # nothing was detached from the module on the way
    assert all(isinstance(p, torch.nn.Parameter) for _, p in named)


def test_norm_weights_of_plain_parameters_and_refusals():
    """``tests/unit/test_single_process_components.py:347-362``, ``:408-416``: a replicated
    parameter weighs 1/W (0.25 at W=4), a parameter split 2 ways over 4 ranks weighs 2/4,
    a world size of 0 and an optimizer over no parameters are refused."""
    from hybrid_training_amd import OptimizerConfig, ShardingError, build_gradient_norm_contributions
    from hybrid_training_amd.optim import build_inner_optimizer

    replicated = torch.nn.Parameter(torch.ones(4))
    assert build_gradient_norm_contributions([replicated], world_size=4)[0].scale == pytest.approx(0.25)
    split = torch.nn.Parameter(torch.ones(4))
    split.is_tensor_parallel_replicated = False
    split.tensor_parallel_group_size = 2
    assert build_gradient_norm_contributions([split], world_size=4)[0].scale == pytest.approx(0.5)
    with pytest.raises(ShardingError, match="world_size must be positive"):
        build_gradient_norm_contributions([torch.nn.Parameter(torch.ones(1))], world_size=0)
    with pytest.raises(ShardingError, match="no trainable parameters"):
        build_inner_optimizer([], OptimizerConfig())


def test_pending_unscale_factors_are_applied_once_per_group(monkeypatch):
    """``_apply_pending_unscale`` (a second deferred ``unscale_``, or a step handed to an
    optimizer that does not read deferred factors): one in-place scaling per (device,
    dtype, factor) group, each gradient's factor dropped afterwards, gradients without a
    factor left alone.  The native scaling is recorded instead of run."""
    from hybrid_training_amd import grad_scaler
    from hybrid_training_amd.optim import PENDING_UNSCALE_ATTR

    calls = []
    monkeypatch.setattr(grad_scaler, "scale_gradients",
                        lambda grads, dtype, factor, mul, device, op: calls.append(
                            (tuple(id(g) for g in grads), dtype, factor, mul, str(device))))
    a, b, c = torch.zeros(3), torch.zeros(4), torch.zeros(5, dtype=torch.bfloat16)
    d, untouched = torch.zeros(2), torch.zeros(6)
    for g, factor in ((a, 0.5), (b, 0.5), (c, 0.5), (d, 0.25)):
        setattr(g, PENDING_UNSCALE_ATTR, factor)
    grad_scaler._apply_pending_unscale([a, None, b, c, d, untouched], torch.device("cuda", 0))
    assert sorted(calls, key=lambda x: (str(x[1]), x[2])) == sorted([
        ((id(a), id(b)), torch.float32, 0.5, None, "cuda:0"),
        ((id(c),), torch.bfloat16, 0.5, None, "cuda:0"),
        ((id(d),), torch.float32, 0.25, None, "cuda:0"),
    ], key=lambda x: (str(x[1]), x[2]))
    assert not any(hasattr(g, PENDING_UNSCALE_ATTR) for g in (a, b, c, d, untouched))
    calls.clear()
    grad_scaler._apply_pending_unscale([a, b], torch.device("cuda", 0))  # nothing pending: no call
    assert calls == []
    # a strided gradient is refused before anything is scaled, the dense one included
    from hybrid_training_amd import ShardingError

    dense, strided = torch.zeros(4), torch.zeros(8)[::2]
    for g in (dense, strided):
        setattr(g, PENDING_UNSCALE_ATTR, 0.5)
    with pytest.raises(ShardingError, match="dense"):
        grad_scaler._apply_pending_unscale([dense, strided], torch.device("cuda", 0))
    assert calls == [] and hasattr(dense, PENDING_UNSCALE_ATTR)


def test_norm_partials_follow_the_version_counter_not_the_data():
    """A gradient's cached norm partials are keyed by its address, dtype and autograd
    version.  Any in-place torch op, and every kernel of this package that writes a tensor
    (``_native.bump_versions``), moves the version and drops them; a write through
    ``tensor.data`` bypasses the counter, so the stale partials are still returned: the
    documented limit of the cache."""
    from hybrid_training_amd import _native
    from hybrid_training_amd.optim import NORM_PARTIALS_ATTR, NormPartials

    g = torch.ones(8)
    partials = torch.tensor([8.0], dtype=torch.float64)
    setattr(g, NORM_PARTIALS_ATTR, NormPartials(g.data_ptr(), g._version, {(0, 8): partials}, g.dtype))
    record = getattr(g, NORM_PARTIALS_ATTR)
    assert record.lookup(g, 0, 8) is partials
    g.data.mul_(2.0)  # no version bump: the cache cannot see it
    assert record.lookup(g, 0, 8) is partials
    _native.bump_versions([g])  # what a kernel writing g does
    assert record.lookup(g, 0, 8) is None
    h = torch.ones(8)
    setattr(h, NORM_PARTIALS_ATTR, NormPartials(h.data_ptr(), h._version, {(0, 8): partials}, h.dtype))
    h.mul_(2.0)
    assert getattr(h, NORM_PARTIALS_ATTR).lookup(h, 0, 8) is None
    with torch.inference_mode():
        frozen = torch.ones(2)
    _native.bump_versions([frozen])  # inference tensors have no counter: skipped, no error


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16, torch.int64])
def test_step_counter_advances_as_torch_adds_one(dtype):
    """The AdamW step counter is advanced on the host (the value, then fill_): the value
    must be what torch's ``step_t += 1`` stores, counts where float32 rounds included."""
    from hybrid_training_amd.optim import _next_step

    rng = np.random.default_rng(5)
    counts = [0.0, 1.0, 2.0**24 - 1, 2.0**24, 2.0**24 + 2, 2.0**25 + 4, 3e7, 1e30, 2.0**127, -5.0, 0.5]
    counts += list(rng.uniform(0, 2**26, 2000)) + list(np.floor(rng.uniform(0, 2**30, 2000)))
    for value in counts:
        if dtype == torch.float16 and abs(value) > 60000:
            continue
        if dtype == torch.int64 and (value != int(value) or abs(value) > 2**62):
            continue
        counter = torch.tensor(value, dtype=dtype)
        expected = counter.clone()
        expected += 1
        got = _next_step(counter)
        counter.fill_(got)
        assert torch.equal(counter, expected) and got == float(expected.item()), (dtype, value)


def test_gradient_signature_of_a_full_bucket_pack():
    """The key under which a full DDP pack reuses its launches: every gradient's address,
    dtype and element count, and no key at all when a gradient is missing or strided
    (such a pack goes through the checks and temporary dense copies every time)."""
    from hybrid_training_amd.buckets import _gradient_signature

    params = [torch.nn.Parameter(torch.zeros(s)) for s in ((3, 4), (5,), (2, 2, 2))]
    for p in params:
        p.grad = torch.randn(p.shape)
    ptrs, dtypes, numels = _gradient_signature(params)
    assert ptrs == tuple(p.grad.data_ptr() for p in params)
    assert dtypes == (torch.float32,) * 3 and numels == (12, 5, 8)
    again = _gradient_signature(params)
    assert again == (ptrs, dtypes, numels)
    params[1].grad = torch.randn(5)  # another tensor: another address
    assert _gradient_signature(params)[0] != ptrs
    params[0].grad = torch.randn(4, 3).t()  # strided
    assert _gradient_signature(params) is None
    params[0].grad = torch.randn(3, 4)
    params[2].grad = None  # missing
    assert _gradient_signature(params) is None
