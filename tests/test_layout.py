"""Flat-buffer layout, shard sizing and interval arithmetic (host logic, no GPU).

Known answers are the reference's own (``tests/unit/test_tensor_utils.py``,
``tests/distributed/test_fsdp.py:42-46, 373-399``, ``README.md:106-107``) plus the
model sizes the benchmark configurations name.  The oracle's restatement is pinned
against the same answers, and the product's functions against both.
"""

from __future__ import annotations

import itertools

import pytest
import torch

import oracle
from hybrid_training_amd import (
    ShardingError,
    ShardRange,
    build_flat_layout,
    concat_shard_sizes,
    even_shard_ranges,
    intersect_ranges,
    shard_range_for,
    unflatten_to_views,
)
from hybrid_training_amd.tensors import bytes_of, numel_of

from .model_shapes import LLAMA3_8B, LLAMA3_70B_TOTAL, MLP_23_32_32_1, MLP_1857_REFERENCE


def test_documented_layout_example():
    entries, total = build_flat_layout(
        [("p0", torch.zeros(2, 3)), ("p1", torch.zeros(4)), ("p2", torch.zeros(3, 2))]
    )
    assert total == 16
    assert [(e.name, e.offset, e.numel) for e in entries] == [("p0", 0, 6), ("p1", 6, 4), ("p2", 10, 6)]
    assert entries[2].end == 16
    assert oracle.flat_layout([6, 4, 6]) == ([0, 6, 10], 16)


def test_layout_errors():
    with pytest.raises(ShardingError, match="duplicate tensor name"):
        build_flat_layout([("w", torch.zeros(2)), ("w", torch.zeros(2))])
    with pytest.raises(ShardingError, match="cannot flatten an empty tensor list"):
        build_flat_layout([])
    entries, _ = build_flat_layout([("a", torch.zeros(8))])
    with pytest.raises(ShardingError, match="too short"):
        unflatten_to_views(torch.zeros(4), entries)
    with pytest.raises(ShardingError, match="one-dimensional"):
        unflatten_to_views(torch.zeros(2, 2), entries)


def test_views_alias_the_flat_buffer():
    entries, _ = build_flat_layout([("a", torch.zeros(2, 2)), ("b", torch.zeros(3))])
    flat = torch.zeros(7)
    views = unflatten_to_views(flat, entries)
    views[0][0, 0] = 5.0
    views[1][2] = 9.0
    assert flat[0].item() == 5.0 and flat[6].item() == 9.0


@pytest.mark.parametrize(("numel", "multiple", "padded"), [(10, 4, 12), (8, 4, 8), (1, 3, 3), (7, 1, 7), (0, 4, 0)])
def test_padding_sizes(numel, multiple, padded):
    assert concat_shard_sizes(numel, multiple)[0] == padded
    shard, total, pad = oracle.even_shards(numel, multiple)
    assert total == padded and pad == padded - numel


def test_shard_ranges_known_answers():
    assert [r.as_tuple() for r in even_shard_ranges(10, 4)] == [(0, 3), (3, 3), (6, 3), (9, 3)]
    assert shard_range_for(10, 4, 2).as_tuple() == (6, 3)
    with pytest.raises(ShardingError, match="shard index outside the group"):
        shard_range_for(10, 4, 4)
    with pytest.raises(ShardingError, match="num_shards must be positive"):
        even_shard_ranges(8, 0)
    with pytest.raises(ShardingError, match="non-negative"):
        ShardRange(start=-1, length=4)
    for numel in range(1, 40):
        for shards in range(1, 7):
            ranges = even_shard_ranges(numel, shards)
            assert len({r.length for r in ranges}) == 1
            for a, b in itertools.pairwise(ranges):
                assert a.end == b.start


@pytest.mark.parametrize(
    ("a", "b", "expected"),
    [((0, 6), (4, 6), (4, 2)), ((0, 4), (4, 4), None), ((0, 10), (2, 3), (2, 3)), ((5, 5), (0, 3), None),
     ((0, 3), (0, 3), (0, 3)), ((3, 0), (0, 10), None)],
)
def test_intersections(a, b, expected):
    got = intersect_ranges(ShardRange(*a), ShardRange(*b))
    assert (None if got is None else got.as_tuple()) == expected


def test_reshard_scenario_from_the_reference():
    saved = even_shard_ranges(12, 4)
    wanted = even_shard_ranges(12, 3)
    table = [[intersect_ranges(s, w).as_tuple() for s in saved if intersect_ranges(s, w)] for w in wanted]
    assert table == [[(0, 3), (3, 1)], [(4, 2), (6, 2)], [(8, 1), (9, 3)]]


@pytest.mark.parametrize("shapes", [MLP_1857_REFERENCE, MLP_23_32_32_1])
def test_1857_parameter_mlp_shards(shapes):
    numels = [int(torch.Size(s).numel()) for s in shapes]
    _, total = oracle.flat_layout(numels)
    assert total == 1857
    assert oracle.even_shards(total, 2) == (929, 1858, 1)
    assert oracle.even_shards(total, 4) == (465, 1860, 3)
    assert concat_shard_sizes(total, 2) == (1858, 929)
    assert concat_shard_sizes(total, 4) == (1860, 465)


def test_llama_shard_sizes():
    numels = [int(torch.Size(s).numel()) for _, s in LLAMA3_8B]
    assert len(numels) == 291
    total = sum(numels)
    assert total == 8_030_261_248
    assert oracle.even_shards(total, 8) == (1_003_782_656, total, 0)
    assert oracle.even_shards(total, 4) == (2_007_565_312, total, 0)
    assert oracle.even_shards(total, 2) == (4_015_130_624, total, 0)
    assert oracle.even_shards(total, 3) == (2_676_753_750, total + 2, 2)
    assert oracle.even_shards(LLAMA3_70B_TOTAL, 8)[0] == 8_819_213_312


def test_measurement_helpers():
    named = [("a", torch.zeros(2, 3)), ("b", torch.zeros(4, dtype=torch.float64))]
    assert numel_of(named) == 10
    assert bytes_of([t for _, t in named]) == 6 * 4 + 4 * 8
