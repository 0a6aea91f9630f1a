"""Shard records and interval lookup (host logic, no GPU).

Known answers from ``tests/unit/test_checkpoint_format.py:150-269`` of the reference.
"""

from __future__ import annotations

import pytest

import numpy as np

import oracle
from hybrid_training_amd import ShardRange, ShardRecord, TensorRecord, shard_filename
from hybrid_training_amd.errors import CheckpointCorruptionError, CheckpointError, IncompleteCheckpointError


def _record(shards, shape=(3, 4)):
    rec = TensorRecord(key="w", name="w", global_shape=shape, dtype="torch.float32")
    rec.shards = [ShardRecord(rank=r, file=shard_filename(r), offset=o, length=n, key=f"model::w@{o}")
                  for r, o, n in shards]
    return rec


def test_complete_record_validates():
    _record([(0, 0, 3), (1, 3, 3), (2, 6, 3), (3, 9, 3)]).validate()


def test_gap_overlap_and_past_end_are_detected():
    with pytest.raises(IncompleteCheckpointError, match="do not cover the whole tensor"):
        _record([(0, 0, 3), (2, 6, 3), (3, 9, 3)]).validate()
    with pytest.raises(CheckpointCorruptionError, match="overlap"):
        _record([(0, 0, 6), (1, 3, 3), (2, 6, 6)]).validate()
    with pytest.raises(CheckpointCorruptionError, match="runs past the end"):
        _record([(0, 0, 12), (1, 12, 4)]).validate()


def test_covered_elements_is_a_union():
    rec = TensorRecord(key="w", name="w", global_shape=(12,), dtype="torch.float32")
    rec.shards = [
        ShardRecord(rank=0, file="rank-00000.pt", offset=0, length=8, key="a"),
        ShardRecord(rank=1, file="rank-00001.pt", offset=4, length=8, key="b"),
    ]
    assert rec.covered_elements() == 12
    assert sum(s.length for s in rec.shards) == 16


def test_shards_overlapping_known_answer():
    rec = _record([(0, 0, 3), (1, 3, 3), (2, 6, 3), (3, 9, 3)])
    got = rec.shards_overlapping(ShardRange(start=0, length=4))
    assert [(s.rank, o.as_tuple()) for s, o in got] == [(0, (0, 3)), (1, (3, 1))]
    assert _record([(0, 0, 3)]).shards_overlapping(ShardRange(start=8, length=2)) == []


def test_round_trip_and_filename_rule():
    rec = _record([(0, 0, 6), (1, 6, 6)])
    again = TensorRecord.from_dict(rec.as_dict())
    assert again == rec
    for bad in ("../../etc/passwd", "/etc/shadow", "rank-1.pt", "rank-00001.pth"):
        with pytest.raises(CheckpointError, match="shard naming rule"):
            ShardRecord(rank=0, file=bad, offset=0, length=1, key="k")
    with pytest.raises(CheckpointError, match="non-negative"):
        ShardRecord(rank=0, file="rank-00000.pt", offset=-1, length=1, key="k")


def test_oracle_read_range_known_answers():
    data = np.arange(12, dtype=np.float32)
    pieces = [(o, data[o : o + 3]) for o in (0, 3, 6, 9)]
    for start, length in ((0, 4), (4, 4), (8, 4), (0, 12), (5, 1)):
        assert np.array_equal(oracle.read_range(pieces, start, length), data[start : start + length])
    with pytest.raises(ValueError, match="gap"):
        oracle.read_range([pieces[0], pieces[2]], 0, 9)
