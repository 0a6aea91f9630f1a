"""GPU parity of checkpoint resharding (``read_tensor_range``, ``load_flat_shard``).

Small cases follow the reference's known answers and error paths
(``tests/unit/test_tensor_utils.py:219-230``, ``checkpoint/reshard.py:224-302``).  The
full-size case is Llama-3-8B in bf16 (8,030,261,248 elements, 291 tensors) saved as
per-tensor shard records by 4 writers and loaded by 2, 8 and 3 readers; every
destination shard must equal the matching slice of the global flat vector bitwise,
and the W=3 padding tail must stay untouched.
"""

from __future__ import annotations

import pytest
import torch

from hybrid_training_amd import (
    DeviceShardCache,
    PieceLayout,
    ShardRange,
    ShardRecord,
    TensorRecord,
    intersect_ranges,
    load_flat_shard,
    read_tensor_range,
    shard_filename,
)
from hybrid_training_amd.errors import CheckpointCorruptionError, CheckpointError, IncompleteCheckpointError

from .model_shapes import LLAMA3_8B

pytestmark = pytest.mark.gpu


def _numel(shape):
    n = 1
    for s in shape:
        n *= s
    return n


def _save(named_shapes, shards, shard_numel, dtype_str):
    """Per-tensor records and a device cache for flat shards written by len(shards) ranks."""
    records: dict[str, TensorRecord] = {}
    cache = DeviceShardCache()
    cursor = 0
    for name, shape in named_shapes:
        numel = _numel(shape)
        rec = TensorRecord(key=name, name=name, global_shape=tuple(shape), dtype=dtype_str)
        for rank, shard in enumerate(shards):
            ov = intersect_ranges(ShardRange(rank * shard_numel, shard_numel), ShardRange(cursor, numel))
            if ov is None:
                continue
            key = f"model::{name}@{ov.start - cursor}"
            rec.shards.append(ShardRecord(rank=rank, file=shard_filename(rank), offset=ov.start - cursor,
                                          length=ov.length, key=key))
            cache.add(shard_filename(rank), key, shard[ov.start - rank * shard_numel : ov.end - rank * shard_numel])
        rec.validate()
        records[name] = rec
        cursor += numel
    return records, cache


def _layout(named_shapes, rank, shard_numel):
    local = ShardRange(rank * shard_numel, shard_numel)
    out, cursor = [], 0
    for name, shape in named_shapes:
        numel = _numel(shape)
        ov = intersect_ranges(local, ShardRange(cursor, numel))
        if ov is not None:
            out.append(PieceLayout(name=name, global_shape=tuple(shape), parameter_offset=ov.start - cursor,
                                   length=ov.length, local_offset=ov.start - local.start))
        cursor += numel
    return out


def test_four_writers_three_readers(device):
    data = torch.arange(12, dtype=torch.float32, device=device)
    shards = [data[3 * r : 3 * r + 3].clone() for r in range(4)]
    records, cache = _save([("w", (3, 4))], shards, 3, "torch.float32")
    for r, (start, length) in enumerate(((0, 4), (4, 4), (8, 4))):
        got = read_tensor_range(records["w"], ShardRange(start, length), cache)
        assert torch.equal(got, data[start : start + length])
        dest = torch.full((4,), -1.0, device=device)
        assert load_flat_shard(dest, _layout([("w", (3, 4))], r, 4), records, cache) == 1
        assert torch.equal(dest, data[start : start + length])
    assert cache.loaded_files() == tuple(shard_filename(r) for r in range(4))
    as_bf16 = read_tensor_range(records["w"], ShardRange(2, 7), cache, dtype=torch.bfloat16)
    assert torch.equal(as_bf16, data[2:9].to(torch.bfloat16))
    assert read_tensor_range(records["w"], ShardRange(5, 0), cache).numel() == 0


def test_error_paths(device):
    data = torch.arange(12, dtype=torch.float32, device=device)
    shards = [data[3 * r : 3 * r + 3].clone() for r in range(4)]
    records, cache = _save([("w", (3, 4))], shards, 3, "torch.float32")
    rec = records["w"]
    with pytest.raises(CheckpointError, match="past the end"):
        read_tensor_range(rec, ShardRange(10, 5), cache)
    gap = TensorRecord(key="w", name="w", global_shape=(3, 4), dtype="torch.float32",
                       shards=[rec.shards[0], rec.shards[2]])
    with pytest.raises(IncompleteCheckpointError, match="gap"):
        read_tensor_range(gap, ShardRange(0, 9), cache)
    none = TensorRecord(key="w", name="w", global_shape=(3, 4), dtype="torch.float32", shards=[rec.shards[0]])
    with pytest.raises(IncompleteCheckpointError, match="none of the saved intervals"):
        read_tensor_range(none, ShardRange(6, 3), cache)
    with pytest.raises(IncompleteCheckpointError, match="supply"):
        read_tensor_range(none, ShardRange(0, 6), cache)
    wrong_key = TensorRecord(key="w", name="w", global_shape=(3, 4), dtype="torch.float32",
                             shards=[ShardRecord(rank=0, file="rank-00000.pt", offset=0, length=12, key="nope")])
    with pytest.raises(CheckpointCorruptionError, match="holds no entry"):
        read_tensor_range(wrong_key, ShardRange(0, 4), cache)
    wrong_len = TensorRecord(key="w", name="w", global_shape=(3, 4), dtype="torch.float32",
                             shards=[ShardRecord(rank=0, file="rank-00000.pt", offset=0, length=12,
                                                 key=rec.shards[0].key)])
    with pytest.raises(CheckpointCorruptionError, match="its record says"):
        read_tensor_range(wrong_len, ShardRange(0, 4), cache)
    missing = TensorRecord(key="w", name="w", global_shape=(3, 4), dtype="torch.float32",
                           shards=[ShardRecord(rank=9, file="rank-00009.pt", offset=0, length=12, key="k")])
    with pytest.raises(IncompleteCheckpointError, match="missing"):
        read_tensor_range(missing, ShardRange(0, 4), cache)
    with pytest.raises(IncompleteCheckpointError, match="no tensor"):
        load_flat_shard(torch.zeros(4, device=device), _layout([("v", (4,))], 0, 4), records, cache)


def test_llama3_8b_bf16_reshard_full_size(device):
    total = sum(_numel(s) for _, s in LLAMA3_8B)
    assert total == 8_030_261_248
    w_src = 4
    s_src = total // w_src
    gen = torch.Generator(device=device).manual_seed(4)
    shards = [torch.randint(-(2**15), 2**15, (s_src,), dtype=torch.int16, device=device, generator=gen)
              .view(torch.bfloat16) for _ in range(w_src)]
    records, cache = _save(LLAMA3_8B, shards, s_src, "torch.bfloat16")

    def global_slice(start, length):
        """Concatenation of the source shards restricted to [start, start + length)."""
        parts, cursor = [], start
        while cursor < start + length:
            r, off = divmod(cursor, s_src)
            n = min(s_src - off, start + length - cursor)
            parts.append(shards[r][off : off + n])
            cursor += n
        return parts

    for w_dst in (8, 2, 3):
        s_dst = -(-total // w_dst)
        dest = torch.zeros(s_dst, dtype=torch.bfloat16, device=device)
        for rank in range(w_dst):
            dest.view(torch.int16).fill_(0)
            layout = _layout(LLAMA3_8B, rank, s_dst)
            assert load_flat_shard(dest, layout, records, cache) == len(layout)
            valid = min(s_dst, total - rank * s_dst)
            cursor = 0
            for part in global_slice(rank * s_dst, valid):
                assert torch.equal(dest[cursor : cursor + part.numel()].view(torch.int16), part.view(torch.int16))
                cursor += part.numel()
            if valid < s_dst:
                assert int(dest[valid:].view(torch.int16).abs().sum()) == 0
        del dest
        torch.cuda.empty_cache()
