"""GPU parity of the FSDP flat parameter: pack/pad/shard, unpack, pieces, gradient share.

The 1857-parameter MLPs of the reference tests (``test_fsdp.py:42-46``) at group sizes
1, 2, 3 and 4 cover padding of 0, 1, 2 and 3 elements; every rank's shard, piece set
and gradient share is checked bitwise against the oracle's restatement
(``oracle.pack_shard``, ``oracle.local_share``) and against the reference's
invariants: padding is exactly 0.0 in parameters and gradients, pieces cover every
parameter once, and ``full_tensors`` reproduces the originals bitwise.  ``no_sync``
accumulation is checked against the oracle's restatement of the reference's
clone/add_/add sequence followed by its local share.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import (
    FlatParamHandle,
    FSDPConfig,
    GroupHandle,
    MixedPrecisionConfig,
    ShardedTensorPiece,
    ShardingError,
    optimizer_parameter_layout,
    reshard_state_dict_pieces,
)
from hybrid_training_amd.errors import UnsupportedFeatureError
from hybrid_training_amd.optim import NORM_PARTIALS_ATTR

from .model_shapes import MLP_23_32_32_1, MLP_1857_REFERENCE

pytestmark = pytest.mark.gpu


def _params(shapes, device, seed=3, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    return [(f"p{i}", torch.nn.Parameter((torch.randn(s, generator=gen) * 0.1).to(dtype).to(device)))
            for i, s in enumerate(shapes)]


def _handles(shapes, group, device, **kw):
    named = _params(shapes, device)
    originals = [p.detach().clone() for _, p in named]
    handles = [
        FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(),
                        MixedPrecisionConfig(), device, keep_originals=True, **kw)
        for r in range(group)
    ]
    return named, originals, handles


@pytest.mark.parametrize("shapes", [MLP_1857_REFERENCE, MLP_23_32_32_1])
@pytest.mark.parametrize("group", [1, 2, 3, 4])
def test_pack_pad_shard_matches_oracle(device, shapes, group):
    named, originals, handles = _handles(shapes, group, device)
    host = [o.cpu().numpy() for o in originals]
    shard, padded, pad = oracle.even_shards(1857, group)
    for rank, h in enumerate(handles):
        assert (h.total_numel, h.shard_numel, h.padded_numel, h.padding) == (1857, shard, padded, pad)
        assert h.local_shard_range().as_tuple() == (rank * shard, shard)
        expect = oracle.pack_shard(host, group, rank)
        assert np.array_equal(h.flat_param.detach().cpu().numpy().view(np.int32), expect.view(np.int32))
        assert h.memory_summary()["padding_bytes"] == pad * 4
    # pieces cover every parameter exactly once across the group
    owned = sum(item.length for h in handles for item in h.local_piece_layout())
    assert owned == 1857
    full = handles[0].full_tensors(peer_shards=[h.flat_param for h in handles])
    for (name, _), orig in zip(named, originals):
        assert torch.equal(full[name], orig)
    pieces = [p for h in handles for p in h.local_pieces()]
    for (name, _), orig in zip(named, originals):
        mine = [p for p in pieces if p.name == name]
        assert torch.equal(reshard_state_dict_pieces(mine, tuple(orig.shape)), orig)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_reshard_state_dict_pieces_overlapping_pieces_last_writer_wins(device, seed):
    """``parallel/fsdp.py:1670-1730`` assigns the pieces' slices in list order, so where
    pieces overlap the later one's values stand.  The expected tensor is that sequential
    assignment done on the CPU; pieces start at odd offsets (misaligned sources and
    destinations) and one piece's data is a non-contiguous view."""
    rng = np.random.default_rng(seed)
    shape = (37, 29)
    total = shape[0] * shape[1]
    spans = [(0, total // 2 + 5), (total // 2 - 11, total - total // 2 + 11)]
    for _ in range(5):
        start = int(rng.integers(0, total - 1))
        spans.append((start, int(rng.integers(1, total - start + 1))))
    order = rng.permutation(len(spans))
    spans = [spans[i] for i in order]
    expected = torch.full((total,), float("nan"))
    pieces = []
    for k, (offset, length) in enumerate(spans):
        values = torch.arange(length, dtype=torch.float32) + 1000.0 * (k + 1)
        expected[offset:offset + length] = values
        data = values.to(device)
        if k == 1:
            wide = torch.empty((length, 2), device=device)
            wide[:, 0] = data
            data = wide[:, 0]
            assert not data.is_contiguous()
        pieces.append(ShardedTensorPiece(name="w", global_shape=shape, offset=offset, data=data))
    assert not torch.isnan(expected).any()
    got = reshard_state_dict_pieces(pieces, shape)
    assert got.shape == shape
    assert torch.equal(got.reshape(-1).cpu().view(torch.int32), expected.view(torch.int32))
    with pytest.raises(ShardingError, match="lie in none of the given pieces"):
        reshard_state_dict_pieces([p for p in pieces if p.offset != 0], shape)
    with pytest.raises(ShardingError, match="past the end"):
        reshard_state_dict_pieces(pieces + [ShardedTensorPiece(name="w", global_shape=shape, offset=total - 2,
                                                               data=torch.zeros(3, device=device))], shape)


def test_optimizer_parameter_layout_prefixes_each_units_pieces(device):
    """``fsdp.py:1477-1510``: every unit's flat shard with its local pieces, the piece
    names carrying the unit's prefix and everything else as ``local_piece_layout``."""
    _, _, first = _handles(MLP_1857_REFERENCE, 2, device)
    _, _, second = _handles(MLP_23_32_32_1, 3, device)
    units = [("layers.0.", first[1]), ("layers.1.", second[2])]
    layout = optimizer_parameter_layout(units)
    assert len(layout) == 2 and all(p is h.flat_param for (p, _), (_, h) in zip(layout, units))
    for (prefix, h), (_, pieces) in zip(units, layout):
        plain = h.local_piece_layout()
        assert [p.name for p in pieces] == [prefix + q.name for q in plain]
        assert [(p.global_shape, p.parameter_offset, p.length, p.local_offset) for p in pieces] == \
            [(q.global_shape, q.parameter_offset, q.length, q.local_offset) for q in plain]
        assert sum(p.length for p in pieces) <= h.shard_numel


def test_build_and_load_from_host_tensors(device):
    """Parameters and state-dict tensors on the host are uploaded tensor by tensor, and
    each upload (and each dense copy of a non-contiguous tensor) must stay alive until
    the copy that reads it has run; a dropped one would hand its memory to the next
    upload first.  Shards bitwise against the oracle."""
    gen = torch.Generator().manual_seed(21)
    named = [(f"p{i}", torch.nn.Parameter(torch.randn(s, generator=gen))) for i, s in enumerate(MLP_1857_REFERENCE)]
    host = [p.detach().numpy().copy() for _, p in named]
    for group in (1, 3):
        for rank in range(group):
            h = FlatParamHandle(named, None, GroupHandle.local_view("shard", group, rank), FSDPConfig(),
                                MixedPrecisionConfig(), device, keep_originals=True)
            expect = oracle.pack_shard(host, group, rank)
            assert np.array_equal(h.flat_param.detach().cpu().numpy().view(np.int32), expect.view(np.int32))
            state = {}
            for name, p in named:
                if p.dim() == 2:  # a transposed view: non-contiguous
                    state[name] = torch.randn(tuple(reversed(p.shape)), generator=gen).t()
                else:
                    state[name] = torch.randn(p.shape, generator=gen)
            h.load_local_pieces(state)
            expect = oracle.pack_shard([state[name].contiguous().numpy() for name, _ in named], group, rank)
            assert np.array_equal(h.flat_param.detach().cpu().numpy().view(np.int32), expect.view(np.int32))


def test_padding_only_ranks_and_empty_parameters(device):
    """Three one-element parameters and an empty one over 8 ranks: ranks 3-7 hold only
    padding.  Every rank's shard, pieces, gathered tensors, local share and no_sync
    result follow the reference's layout rules, bitwise against the oracle."""
    values = [torch.tensor([1.5], device=device), torch.empty(0, device=device),
              torch.tensor([-2.25], device=device), torch.tensor([0.75], device=device)]
    named = [(f"t{i}", torch.nn.Parameter(v.clone())) for i, v in enumerate(values)]
    group = 8
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(),
                               MixedPrecisionConfig(), device, keep_originals=True) for r in range(group)]
    host = [v.cpu().numpy() for v in values]
    assert (handles[0].total_numel, handles[0].shard_numel, handles[0].padding) == (3, 1, 5)
    for rank, h in enumerate(handles):
        expect = oracle.pack_shard(host, group, rank)
        assert np.array_equal(h.flat_param.detach().cpu().numpy().view(np.int32), expect.view(np.int32))
        assert [p.name for p in h.local_piece_layout()] == ([["t0"], ["t2"], ["t3"]][rank] if rank < 3 else [])
    full = handles[0].full_tensors(peer_shards=[h.flat_param for h in handles])
    for (name, _), v in zip(named, values):
        assert torch.equal(full[name], v) and full[name].shape == v.shape
    gen = torch.Generator(device=device).manual_seed(2)
    micro = [[torch.randn(group, device=device, generator=gen) for _ in range(group)] for _ in range(2)]
    for rank, h in enumerate(handles):
        out = h.reduce_scatter_gradient(micro[0][rank], peer_grads=micro[0])
        expect = oracle.local_share([g.cpu().numpy() for g in micro[0]], rank, 1, 1 if rank < 3 else 0, 8.0)
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32))
        h.set_accumulate_without_reduction(True)
        assert h.reduce_scatter_gradient(micro[0][rank], peer_grads=micro[0]) is None
        h.set_accumulate_without_reduction(False)
        out = h.reduce_scatter_gradient(micro[1][rank], peer_grads=micro[1])
        totals = [oracle.no_sync_accumulate([micro[m][q].cpu().numpy() for m in range(2)]) for q in range(group)]
        expect = oracle.local_share(totals, rank, 1, 1 if rank < 3 else 0, 8.0)
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32))


def test_norm_weights_and_padding_runs(device):
    _, _, handles = _handles(MLP_1857_REFERENCE, 4, device)
    last = handles[-1]
    runs = last.flat_param.gradient_norm_scale_runs
    assert runs[-1] == (465 - 3, 3, 0.0)
    vector = last.flat_param.gradient_norm_scale_vector
    assert vector.shape == (465,) and float(vector[-3:].abs().sum()) == 0.0 and float(vector[0]) == 4.0


@pytest.mark.parametrize("group", [1, 2, 3, 4])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_gradient_local_share_matches_oracle(device, group, in_dtype):
    _, _, handles = _handles(MLP_1857_REFERENCE, group, device)
    padded = handles[0].padded_numel
    gen = torch.Generator(device=device).manual_seed(group)
    grads = [(torch.randn(padded, device=device, generator=gen) * 1e-2).to(in_dtype) for _ in range(group)]
    host = [g.float().cpu().numpy() for g in grads]
    for rank, h in enumerate(handles):
        out = h.reduce_scatter_gradient(grads[rank], peer_grads=grads if group > 1 else None)
        valid = max(0, min(h.shard_numel, 1857 - rank * h.shard_numel))
        expect = oracle.local_share(host, rank, h.shard_numel, valid, float(group) if group > 1 else 1.0)
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32))
        assert float(out[valid:].abs().sum()) == 0.0 if valid < h.shard_numel else True
        assert h.reduction_count == 1


def _mp_handles(group, device, reduce):
    named = _params(MLP_1857_REFERENCE, device)
    mp = MixedPrecisionConfig(enabled=True, param_dtype="bfloat16", reduce_dtype=reduce, master_dtype="float32")
    return [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(), mp, device,
                            keep_originals=True) for r in range(group)]


@pytest.mark.parametrize("group", [1, 2, 3, 4])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("reduce", ["bfloat16", "float16", "float64"])
def test_gradient_local_share_in_reduce_dtype_matches_oracle(device, group, in_dtype, reduce):
    """``MixedPrecisionConfig(reduce_dtype=...)``: the cast, the AVG divide and the rank sum
    rounded to bf16 or fp16 (``collectives.py:593-594`` in that dtype), widened to the
    fp32 master; bitwise against the oracle."""
    handles = _mp_handles(group, device, reduce)
    padded = handles[0].padded_numel
    gen = torch.Generator(device=device).manual_seed(group + 7)
    grads = [(torch.randn(padded, device=device, generator=gen) * 3.0).to(in_dtype) for _ in range(group)]
    host = [g.float().cpu().numpy() for g in grads]
    divisor = float(group) if group > 1 else 1.0
    for rank, h in enumerate(handles):
        out = h.reduce_scatter_gradient(grads[rank], peer_grads=grads if group > 1 else None)
        assert out.dtype == torch.float32
        valid = max(0, min(h.shard_numel, 1857 - rank * h.shard_numel))
        expect = oracle.local_share(host, rank, h.shard_numel, valid, divisor, reduce)
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32)), rank
        assert torch.equal(out.to(getattr(torch, reduce)).to(torch.float32), out)  # representable in it


@pytest.mark.parametrize("group", [2, 3])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("reduce", ["float32", "bfloat16", "float16", "float64"])
def test_local_share_with_ieee_specials_matches_oracle(device, group, in_dtype, reduce):
    """IEEE specials in the gradients (+inf, -inf, NaN, -0.0, values past fp16's range
    and inf meeting -inf across ranks) through the local share in every reduce dtype:
    every result bitwise the oracle's, NaNs compared as NaNs (a NaN's bits after bf16
    arithmetic have no single torch pattern)."""
    handles = _mp_handles(group, device, reduce)
    padded, shard = handles[0].padded_numel, handles[0].shard_numel
    gen = torch.Generator(device=device).manual_seed(group + 31)
    grads = []
    for q in range(group):
        g = torch.randn(padded, device=device, generator=gen) * 3.0
        for r in range(group):
            base = r * shard
            g[base + 1] = float("inf")
            g[base + 2] = -float("inf") if q == 0 else float("inf")  # inf meets -inf: NaN
            g[base + 3] = float("nan")
            g[base + 4] = -0.0
            g[base + 5] = 70000.0 * (q + 1)  # past fp16's range once cast
            g[base + 6] = float("nan") if q == group - 1 else 1.0
        grads.append(g.to(in_dtype))
    host = [g.float().cpu().numpy() for g in grads]
    divisor = float(group)
    for rank, h in enumerate(handles):
        out = h.reduce_scatter_gradient(grads[rank], peer_grads=grads).cpu().numpy()
        valid = max(0, min(shard, 1857 - rank * shard))
        expect = oracle.local_share(host, rank, shard, valid, divisor, reduce)
        nan = np.isnan(expect)
        assert np.array_equal(np.isnan(out), nan), rank
        assert np.array_equal(out[~nan].view(np.int32), expect[~nan].view(np.int32)), rank
        assert nan[2] and nan[3] and nan[6] and np.isinf(out[1]) and out[4] == 0.0 and np.signbit(out[4])


def test_reduce_and_master_dtype_limits(device):
    """A bf16 master shard (mixed precision with ``master_dtype="bfloat16"``) packs and
    reduces into bf16; a float64 master packs (the copy kernel converts into float64) and
    reduces in float64 into a float64 gradient shard, padding zero; float64 gradients
    with a narrower reduce dtype are refused up front."""
    named = _params(MLP_1857_REFERENCE, device)
    mp = MixedPrecisionConfig(enabled=True, master_dtype="bfloat16")
    h = FlatParamHandle(named, None, GroupHandle.trivial("shard"), FSDPConfig(), mp, device, keep_originals=True)
    assert h.flat_param.dtype == torch.bfloat16
    flat = torch.cat([p.detach().reshape(-1) for _, p in named])
    assert torch.equal(h.flat_param.detach()[: flat.numel()], flat.to(torch.bfloat16))
    grad = torch.randn(h.padded_numel, device=device)
    out = h.reduce_scatter_gradient(grad)
    assert out.dtype == torch.bfloat16 and torch.equal(out, grad.to(torch.bfloat16))
    mp = MixedPrecisionConfig(enabled=True, reduce_dtype="float64", master_dtype="float64")
    h = FlatParamHandle(named, None, GroupHandle.trivial("shard"), FSDPConfig(), mp, device, keep_originals=True)
    assert torch.equal(h.flat_param.detach()[: flat.numel()], flat.to(torch.float64))
    out = h.reduce_scatter_gradient(grad)
    expect = grad.to(torch.float64)
    expect[h.total_numel:] = 0.0
    assert out.dtype == torch.float64 and torch.equal(out, expect)
    mp = MixedPrecisionConfig(enabled=True, param_dtype="float64", reduce_dtype="float32")
    h = FlatParamHandle(named, None, GroupHandle.trivial("shard"), FSDPConfig(), mp, device, keep_originals=True)
    with pytest.raises(UnsupportedFeatureError, match="float64 gradients are reduced in float64"):
        h.reduce_scatter_gradient(torch.zeros(h.padded_numel, dtype=torch.float64, device=device))


def test_local_share_needs_every_rank(device):
    _, _, handles = _handles(MLP_1857_REFERENCE, 2, device)
    with pytest.raises(UnsupportedFeatureError, match="reduce-scatter needs every rank"):
        handles[0].reduce_scatter_gradient(torch.zeros(handles[0].padded_numel, device=device))
    with pytest.raises(UnsupportedFeatureError, match="needs every rank's shard"):
        handles[0].full_tensors()
    # ... inside no_sync too: accumulation also needs every rank's gradient
    handles[0].set_accumulate_without_reduction(True)
    with pytest.raises(UnsupportedFeatureError, match="reduce-scatter needs every rank"):
        handles[0].reduce_scatter_gradient(torch.zeros(handles[0].padded_numel, device=device))
    assert handles[0].has_pending_accumulation is False


@pytest.mark.parametrize("group", [1, 2, 3, 4])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("micro", [2, 4])
@pytest.mark.parametrize("reduce", ["float32", "bfloat16", "float16", "float64"])
def test_no_sync_accumulation_matches_oracle(device, group, in_dtype, micro, reduce):
    """``no_sync`` (``parallel/fsdp.py:733-749``): the first ``micro - 1`` micro-batches
    accumulate in the reduce dtype and return None; the last reduces the sums.  Bitwise
    against the oracle's local share of the oracle's accumulated gradients, with -0.0
    planted in every rank's slice (a copy, not an add onto zeros, keeps its sign)."""
    handles = _mp_handles(group, device, reduce)
    padded, shard = handles[0].padded_numel, handles[0].shard_numel
    gen = torch.Generator(device=device).manual_seed(100 * group + micro)
    grads = []
    for _ in range(micro):
        batch = []
        for _ in range(group):
            g = (torch.randn(padded, device=device, generator=gen) * 1e-2).to(in_dtype)
            for r in range(group):
                g[r * shard + 5] = -0.0
            batch.append(g)
        grads.append(batch)
    divisor = float(group) if group > 1 else 1.0
    for rank, h in enumerate(handles):
        def micro_batch(m):
            return h.reduce_scatter_gradient(grads[m][rank], peer_grads=grads[m] if group > 1 else None)

        h.set_accumulate_without_reduction(True)
        for m in range(micro - 1):
            assert micro_batch(m) is None
            assert h.has_pending_accumulation
        assert h.reduction_count == 0
        h.set_accumulate_without_reduction(False)
        out = micro_batch(micro - 1)
        assert not h.has_pending_accumulation and h.reduction_count == 1
        totals = [oracle.no_sync_accumulate([grads[m][q].float().cpu().numpy() for m in range(micro)], reduce)
                  for q in range(group)]
        valid = max(0, min(shard, 1857 - rank * shard))
        expect = oracle.local_share(totals, rank, shard, valid, divisor, reduce)
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32)), rank
        assert np.signbit(out[5].item())
        assert getattr(out, NORM_PARTIALS_ATTR, None) is not None
        # the accumulator is gone: the next call reduces its own gradients only
        again = micro_batch(micro - 1)
        plain = oracle.local_share([g.float().cpu().numpy() for g in grads[micro - 1]], rank, shard, valid,
                                   divisor, reduce)
        assert np.array_equal(again.cpu().numpy().view(np.int32), plain.view(np.int32)), rank
        assert h.reduction_count == 2


def test_load_local_pieces_round_trip(device):
    named, originals, handles = _handles(MLP_23_32_32_1, 4, device)
    state = {name: torch.randn_like(orig) for (name, _), orig in zip(named, originals)}
    host = [state[name].cpu().numpy() for name, _ in named]
    for rank, h in enumerate(handles):
        h.load_local_pieces(state)
        assert np.array_equal(h.flat_param.detach().cpu().numpy(), oracle.pack_shard(host, 4, rank))
    full = handles[0].full_tensors(peer_shards=[h.flat_param for h in handles])
    assert all(torch.equal(full[n], state[n]) for n in state)
    with pytest.raises(ShardingError, match="no tensor for parameter"):
        handles[0].load_local_pieces({})
    bad = dict(state)
    bad["p0"] = torch.zeros(3, device=device)
    with pytest.raises(ShardingError, match="another shape"):
        handles[0].load_local_pieces(bad)


def test_mixed_precision_master_cast_and_gather(device):
    named = _params(MLP_1857_REFERENCE, device, dtype=torch.bfloat16)
    mp = MixedPrecisionConfig(enabled=True, param_dtype="bfloat16", reduce_dtype="float32", master_dtype="float32")
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", 2, r), FSDPConfig(), mp, device,
                               keep_originals=True) for r in range(2)]
    host = [p.detach().float().cpu().numpy() for _, p in named]
    for rank, h in enumerate(handles):
        assert h.flat_param.dtype == torch.float32
        assert np.array_equal(h.flat_param.detach().cpu().numpy(), oracle.pack_shard(host, 2, rank))
    full = handles[0].gather_full([h.flat_param for h in handles])
    assert full.dtype == torch.bfloat16 and full.numel() == 1858
    expect = oracle.f32_to_bf16(np.concatenate([oracle.pack_shard(host, 2, r) for r in range(2)]))
    assert np.array_equal(full.view(torch.int16).cpu().numpy().view(np.uint16), expect)


def test_float16_compute_master_cast_gather_and_local_share(device):
    """fp16 compute (the only precision the reference pairs with loss scaling): fp16
    parameters widen exactly into the fp32 master shards, ``gather_full`` narrows the
    masters to fp16 as torch's ``.to(torch.float16)`` does (``fsdp.py:578-579``), and the
    fp16 full gradients widen exactly before the AVG divide (``fsdp.py:734-735``)."""
    named = _params(MLP_1857_REFERENCE, device, dtype=torch.float16)
    mp = MixedPrecisionConfig(enabled=True, param_dtype="float16", reduce_dtype="float32", master_dtype="float32")
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", 2, r), FSDPConfig(), mp, device,
                               keep_originals=True) for r in range(2)]
    host = [p.detach().float().cpu().numpy() for _, p in named]
    for rank, h in enumerate(handles):
        assert h.flat_param.dtype == torch.float32
        assert np.array_equal(h.flat_param.detach().cpu().numpy(), oracle.pack_shard(host, 2, rank))
    # masters that need rounding: scale them off the fp16 grid
    for h in handles:
        h.flat_param.data.mul_(1.0 + 2.0**-13).add_(3e-6)
    full = handles[0].gather_full([h.flat_param for h in handles])
    assert full.dtype == torch.float16 and full.numel() == 1858
    expect = torch.cat([h.flat_param.detach().cpu() for h in handles]).to(torch.float16)
    assert torch.equal(full.cpu().view(torch.int16), expect.view(torch.int16))
    gen = torch.Generator(device=device).manual_seed(16)
    grads = [(torch.randn(1858, device=device, generator=gen) * 1e-2).to(torch.float16) for _ in range(2)]
    host_g = [g.float().cpu().numpy() for g in grads]
    for rank, h in enumerate(handles):
        out = h.reduce_scatter_gradient(grads[rank], peer_grads=grads)
        valid = max(0, min(h.shard_numel, 1857 - rank * h.shard_numel))
        expect_g = oracle.local_share(host_g, rank, h.shard_numel, valid, 2.0)
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect_g.view(np.int32))


def test_detaching_frees_originals_and_binds_views(device):
    module = torch.nn.Linear(4, 3).to(device)
    named = list(module.named_parameters())
    locations = {id(p): [(module, n)] for n, p in named}
    w = module.weight.detach().clone()
    h = FlatParamHandle(named, locations, GroupHandle.trivial(), FSDPConfig(), MixedPrecisionConfig(), device)
    assert "weight" not in module._parameters and module.weight.numel() == 0
    full = h.gather_full()
    h.bind_views(full)
    assert torch.equal(module.weight, w)
    with pytest.raises(ShardingError, match="at least one parameter"):
        FlatParamHandle([], None, GroupHandle.trivial(), FSDPConfig(), MixedPrecisionConfig(), device)


def _wide_model(device):
    """Enough elements for several 32768-element norm chunks per shard, odd total."""
    shapes = [("a", (700, 300)), ("b", (301,)), ("c", (200, 300)), ("d", (9,))]  # 270,310 elements
    gen = torch.Generator(device=device).manual_seed(9)
    return [(n, torch.nn.Parameter(torch.randn(s, device=device, generator=gen))) for n, s in shapes]


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("norm_world", [4, 8])
def test_local_share_norm_partials_are_the_norm_pass(device, in_dtype, norm_world):
    """The fused local share leaves partials that give clip_grad_norm the norm of a
    separate pass over the same shard (within 1e-12 relative: the producer sums in its
    own fixed order), reproducibly, for weight 1 (norm group = shard group) and weight
    1/2 (norm group twice as wide); an in-place change invalidates them."""
    from hybrid_training_amd import GroupHandle, OptimizerConfig, ShardedOptimizer
    from hybrid_training_amd.optim import NORM_PARTIALS_ATTR

    named = _wide_model(device)
    group = 4
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(),
                               MixedPrecisionConfig(), device, keep_originals=True) for r in range(group)]
    total = sum(p.numel() for _, p in named)
    assert handles[-1].padding > 0 and handles[0].shard_numel > 2 * 32768
    gen = torch.Generator(device=device).manual_seed(4)
    grads = [(torch.randn(handles[0].padded_numel, device=device, generator=gen) * 1e-2).to(in_dtype)
             for _ in range(group)]
    host = [g.float().cpu().numpy() for g in grads]
    for rank, h in enumerate(handles):
        assert len(h.flat_param.gradient_norm_scale_runs) <= 2  # merged equal-weight runs
        opt = ShardedOptimizer([h.flat_param], OptimizerConfig(), norm_group=GroupHandle.local_view("world", norm_world, rank),
                               device=device)
        fused = h.reduce_scatter_gradient(grads[rank], peer_grads=grads)
        valid = max(0, min(h.shard_numel, total - rank * h.shard_numel))
        assert getattr(fused, NORM_PARTIALS_ATTR).lookup(fused, 0, valid) is not None
        expect = oracle.local_share(host, rank, h.shard_numel, valid, float(group))
        assert np.array_equal(fused.cpu().numpy().view(np.int32), expect.view(np.int32))
        plain = fused.clone()  # same values, no partials attached
        h.flat_param.grad = plain
        n_plain = opt.clip_grad_norm(0.0)
        h.flat_param.grad = fused
        n_fused = opt.clip_grad_norm(0.0)
        assert abs(float(n_fused) - float(n_plain)) <= 1e-12 * float(n_plain), (rank, float(n_fused), float(n_plain))
        again = h.reduce_scatter_gradient(grads[rank], peer_grads=grads)
        assert torch.equal(again, fused)
        h.flat_param.grad = again
        assert float(opt.clip_grad_norm(0.0)) == float(n_fused)  # reproducible
        h.flat_param.grad = fused
        ref = float((torch.from_numpy(expect).double() ** 2).sum()) * group / norm_world
        assert abs(float(n_fused) ** 2 - ref) <= 1e-12 * ref
        # an in-place change bumps the version counter: the partials are not reused
        fused.mul_(2.0)
        assert float(opt.clip_grad_norm(0.0)) == 2.0 * float(n_plain)


def test_unshard_reshard_refill_free_full_lifecycle(device):
    """The gathered buffer's lifecycle (``fsdp.py:613-701``, ``:783-789``) on a real module:
    unshard binds views, reshard releases the bytes but keeps the tensor and its views,
    refill restores the same bits with the autograd version unchanged, free_full unbinds."""
    module = torch.nn.Linear(25, 14).to(device)
    named = list(module.named_parameters())
    locations = {id(p): [(module, name)] for name, p in named}
    originals = {name: p.detach().clone() for name, p in named}
    mp = MixedPrecisionConfig(enabled=True, param_dtype="bfloat16", reduce_dtype="float32", master_dtype="float32")
    h = FlatParamHandle(named, locations, GroupHandle.trivial("shard"), FSDPConfig(), mp, device)
    assert h.is_sharded
    full = h.unshard()
    assert not h.is_sharded and full.dtype == torch.bfloat16
    assert torch.equal(module.weight, originals["weight"].to(torch.bfloat16))
    assert module.weight.untyped_storage().data_ptr() == full.untyped_storage().data_ptr()
    assert h.memory_summary()["full_bytes"] == full.numel() * 2
    bits = full.detach().clone()
    version = full._version
    h.reshard()
    assert h.is_sharded and full.untyped_storage().nbytes() == 0
    assert h.memory_summary()["full_bytes"] == 0
    h.refill(full)
    assert not h.is_sharded and full._version == version
    assert torch.equal(full.view(torch.int16), bits.view(torch.int16))
    assert torch.equal(module.bias, originals["bias"].to(torch.bfloat16))  # the views see the refilled bytes
    h.refill(full)  # a buffer that holds its storage is left alone
    h.free_full()
    assert h.is_sharded and module.weight.numel() == 0


def test_local_share_at_the_rank_limit(device):
    """``HBT_MAX_LOCAL_RANKS`` (64) ranks on the 1857-parameter MLP (shard 30, padding 63):
    every 8th rank's local share and a two-micro-batch ``no_sync`` end are bitwise the
    oracle's.  With 65 ranks the reduction is refused before any launch: no reduction is
    counted, and a ``no_sync`` accumulation keeps its rows for a retry."""
    from hybrid_training_amd.errors import NativeKernelError

    group = 64
    named = _params(MLP_1857_REFERENCE, device)
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(),
                               MixedPrecisionConfig(), device, keep_originals=True) for r in range(0, group, 8)]
    padded, shard = handles[0].padded_numel, handles[0].shard_numel
    assert shard == 30 and padded - 1857 == 63
    gen = torch.Generator(device=device).manual_seed(64)
    grads = [[torch.randn(padded, device=device, generator=gen) * 1e-2 for _ in range(group)] for _ in range(2)]
    for h, rank in zip(handles, range(0, group, 8)):
        valid = max(0, min(shard, 1857 - rank * shard))
        out = h.reduce_scatter_gradient(grads[0][rank], peer_grads=grads[0])
        expect = oracle.local_share([g.cpu().numpy() for g in grads[0]], rank, shard, valid, float(group))
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32)), rank
        h.set_accumulate_without_reduction(True)
        assert h.reduce_scatter_gradient(grads[0][rank], peer_grads=grads[0]) is None
        h.set_accumulate_without_reduction(False)
        out = h.reduce_scatter_gradient(grads[1][rank], peer_grads=grads[1])
        totals = [oracle.no_sync_accumulate([grads[m][q].cpu().numpy() for m in range(2)], "float32")
                  for q in range(group)]
        expect = oracle.local_share(totals, rank, shard, valid, float(group))
        assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32)), rank
    over = FlatParamHandle(named, None, GroupHandle.local_view("shard", group + 1, 0), FSDPConfig(),
                           MixedPrecisionConfig(), device, keep_originals=True)
    wide = [torch.zeros(over.padded_numel, device=device) for _ in range(group + 1)]
    with pytest.raises(NativeKernelError):
        over.reduce_scatter_gradient(wide[0], peer_grads=wide)
    assert over.reduction_count == 0
    over.set_accumulate_without_reduction(True)
    over.reduce_scatter_gradient(wide[0], peer_grads=wide)
    over.set_accumulate_without_reduction(False)
    with pytest.raises(NativeKernelError):
        over.reduce_scatter_gradient(wide[0], peer_grads=wide)
    assert over.has_pending_accumulation and over.reduction_count == 0
