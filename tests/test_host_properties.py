"""Property tests of the host-side interval arithmetic against brute force (no GPU).

Every kernel launch on the path is driven by integer plans the host builds: flat
offsets and shard ranges, DDP bucket boundaries, checkpoint shard intersections and
manifests, the last-writer segments of a piece reassembly and the copy kernel's
chunk table.
Each property below answers the same question element by element on small inputs
(which tensor owns position i, which shard covers it, which piece wrote it last)
and compares.  A wrong offset, an off-by-one bound or a swapped operand fails on
some generated case.  Hypothesis runs derandomized, so the cases are the same on
every run.
"""

from __future__ import annotations

import bisect
import json

import numpy as np
import pytest
import torch
import torch.nn as nn
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from hybrid_training_amd import (
    CheckpointCorruptionError,
    CheckpointError,
    CheckpointManifest,
    FileRecord,
    IncompleteCheckpointError,
    ShardRange,
    ShardRecord,
    TensorRecord,
    build_buckets,
    build_flat_layout,
    concat_shard_sizes,
    even_shard_ranges,
    intersect_ranges,
    shard_filename,
    shard_range_for,
)
from hybrid_training_amd import reshard as reshard_module
from hybrid_training_amd._native import plan_hints, plan_table
from hybrid_training_amd.flat_param import _last_writer_segments

PROPERTY = settings(derandomize=True, max_examples=300, deadline=None,
                    suppress_health_check=[HealthCheck.too_slow])

RANGES = st.builds(ShardRange, start=st.integers(0, 30), length=st.integers(0, 30))


@PROPERTY
@given(numels=st.lists(st.integers(0, 40), min_size=1, max_size=10), groups=st.integers(1, 9))
def test_flat_layout_and_even_shards_partition_every_element(numels, groups):
    """``utils/tensors.py:137-196, 347-407``; ``collectives.py:894-928``."""
    entries, total = build_flat_layout([(f"t{i}", torch.empty(n)) for i, n in enumerate(numels)])
    owner = np.concatenate([np.full(n, i, dtype=np.int64) for i, n in enumerate(numels)])
    assert total == owner.size
    for i, entry in enumerate(entries):
        positions = np.flatnonzero(owner == i)
        assert entry.numel == positions.size
        # An entry starts after every element of the tensors before it, and its
        # elements are exactly the contiguous run the concatenation gave it.
        assert entry.offset == int((owner < i).sum())
        assert np.array_equal(positions, np.arange(entry.offset, entry.end))
    padded = total
    while padded % groups:
        padded += 1
    assert concat_shard_sizes(total, groups) == (padded, padded // groups)
    ranges = even_shard_ranges(total, groups)
    assert len(ranges) == groups
    hits = np.zeros(padded + 64, dtype=np.int64)
    for index, shard in enumerate(ranges):
        assert shard == shard_range_for(total, groups, index)
        assert shard.length == padded // groups
        hits[shard.start:shard.end] += 1
    assert (hits[:padded] == 1).all() and (hits[padded:] == 0).all()
    assert [r.start for r in ranges] == sorted(r.start for r in ranges)


@PROPERTY
@given(a=RANGES, b=RANGES)
def test_intersect_ranges_is_the_set_intersection(a, b):
    """``utils/tensors.py:410-435``."""
    common = sorted(set(range(a.start, a.end)) & set(range(b.start, b.end)))
    got = intersect_ranges(a, b)
    assert intersect_ranges(b, a) == got
    if not common:
        assert got is None
    else:
        assert got == ShardRange(common[0], len(common))
        assert common == list(range(common[0], common[0] + len(common)))


def _record(numel, shards):
    return TensorRecord(
        key="w", name="w", global_shape=(numel,), dtype="torch.float32",
        shards=[ShardRecord(rank=i, file=f"rank-{i:05d}.pt", offset=o, length=n, key="w")
                for i, (o, n) in enumerate(shards)],
    )


@PROPERTY
@given(numel=st.integers(1, 24),
       shards=st.lists(st.tuples(st.integers(0, 24), st.integers(0, 10)), max_size=6),
       wanted=RANGES)
def test_tensor_record_checks_and_overlaps_match_coverage_counts(numel, shards, wanted):
    """``checkpoint/manifest.py:186-247``: the validation verdict and the intersections
    follow from how many shards cover each element."""
    record = _record(numel, shards)
    count = np.zeros(64, dtype=np.int64)
    for offset, length in shards:
        count[offset:offset + length] += 1
    assert record.covered_elements() == int((count > 0).sum())
    if any(o + n > numel for o, n in shards):
        with pytest.raises(CheckpointCorruptionError, match="past the end"):
            record.validate()
    elif (count > 1).any():
        with pytest.raises(CheckpointCorruptionError, match="overlap"):
            record.validate()
    elif (count[:numel] == 0).any():
        with pytest.raises(IncompleteCheckpointError):
            record.validate()
    else:
        record.validate()

    want = set(range(wanted.start, wanted.end))
    expected = []
    for rank, (offset, length) in sorted(enumerate(shards), key=lambda item: item[1][0]):
        common = sorted(set(range(offset, offset + length)) & want)
        if common:
            expected.append((rank, ShardRange(common[0], len(common))))
    assert [(s.rank, overlap) for s, overlap in record.shards_overlapping(wanted)] == expected


class _HostPayloads:
    """Stands in for the device shard cache: the read planner only calls ``get``."""

    def __init__(self, payloads):
        self.payloads = payloads

    def get(self, filename):
        return self.payloads[filename]


@PROPERTY
@given(numel=st.integers(1, 40),
       cuts=st.lists(st.integers(1, 39), max_size=5, unique=True),
       dropped=st.one_of(st.none(), st.integers(0, 5)),
       start=st.integers(0, 44),
       length=st.integers(1, 20))
def test_read_plan_copies_exactly_the_wanted_elements(numel, cuts, dropped, start, length):
    """``checkpoint/reshard.py:224-302``: a readable range is copied element for element
    from the shards that hold it; a range past the end or with an uncovered element is
    refused with the reference's error class."""
    bounds = sorted({0, numel, *(c for c in cuts if c < numel)})
    pieces = list(zip(bounds[:-1], bounds[1:]))
    skip = None if dropped is None else dropped % len(pieces)
    global_values = np.arange(numel, dtype=np.float32) + 1000.0
    shards, payloads = [], {}
    for rank, (lo, hi) in enumerate(pieces):
        if rank == skip:
            continue
        shards.append((lo, hi - lo))
        payloads[f"rank-{rank:05d}.pt"] = {"w": torch.from_numpy(global_values[lo:hi].copy())}
    record = TensorRecord(
        key="w", name="w", global_shape=(numel,), dtype="torch.float32",
        shards=[ShardRecord(rank=r, file=f"rank-{r:05d}.pt", offset=lo, length=hi - lo, key="w")
                for r, (lo, hi) in enumerate(pieces) if r != skip],
    )
    covered = np.zeros(numel, dtype=bool)
    for offset, n in shards:
        covered[offset:offset + n] = True
    wanted = ShardRange(start, length)
    rows = []

    def plan():
        return reshard_module._queue_range(record, wanted, _HostPayloads(payloads), None, 0,
                                           lambda src, so, do, n: rows.append((src, so, do, n)))

    if wanted.end > numel:
        with pytest.raises(CheckpointError, match="past the end") as info:
            plan()
        assert type(info.value) is CheckpointError
    elif not covered[wanted.start:wanted.end].all():
        with pytest.raises(IncompleteCheckpointError):
            plan()
    else:
        assert plan() == torch.float32
        out = np.full(length, np.nan, dtype=np.float32)
        written = np.zeros(length, dtype=np.int64)
        for src, src_offset, dst_offset, n in rows:
            assert n > 0 and 0 <= src_offset and src_offset + n <= src.numel()
            assert 0 <= dst_offset and dst_offset + n <= length
            out[dst_offset:dst_offset + n] = src.numpy()[src_offset:src_offset + n]
            written[dst_offset:dst_offset + n] += 1
        assert (written == 1).all()
        assert np.array_equal(out.view(np.uint32), global_values[start:start + length].view(np.uint32))


@PROPERTY
@given(spans=st.lists(st.tuples(st.integers(0, 30), st.integers(0, 12)), max_size=7))
def test_last_writer_segments_give_each_element_to_its_last_cover(spans):
    """``parallel/fsdp.py:1670-1730`` places pieces by sequential slice assignment, so
    where pieces overlap the later one wins."""
    intervals = [(s, s + n) for s, n in spans]
    writer = np.full(64, -1, dtype=np.int64)
    for index, (lo, hi) in enumerate(intervals):
        writer[lo:hi] = index
    got = np.full(64, -1, dtype=np.int64)
    for index, lo, hi in _last_writer_segments(intervals):
        assert lo < hi
        assert intervals[index][0] <= lo and hi <= intervals[index][1]
        assert (got[lo:hi] == -1).all(), "segments overlap"
        got[lo:hi] = index
    assert np.array_equal(got, writer)


@PROPERTY
@given(specs=st.lists(st.tuples(st.integers(0, 300), st.sampled_from([torch.float32, torch.bfloat16])),
                      min_size=1, max_size=12),
       data=st.data())
def test_buckets_are_greedy_in_reverse_order_and_split_on_dtype(specs, data):
    """``parallel/ddp.py:397-463``.  The three checks below hold only for the greedy
    partition: every bucket holds one dtype; a bucket of two or more parameters fits
    the cap; and a boundary between same-dtype parameters falls only where the next
    parameter would overflow the bucket.  Half the caps are the exact byte size of a
    run of consecutive parameters, so buckets that fill the cap exactly occur."""
    params = [(f"p{i}", nn.Parameter(torch.empty(n, dtype=dt))) for i, (n, dt) in enumerate(specs)]
    sizes = [p.numel() * p.element_size() for _, p in reversed(params)]
    runs = sorted({sum(sizes[i:j]) for i in range(len(sizes)) for j in range(i + 1, len(sizes) + 1)} - {0})
    caps = st.integers(1, 1500)
    cap_bytes = data.draw(st.one_of(caps, st.sampled_from(runs)) if runs else caps, label="cap_bytes")
    buckets = build_buckets(params, cap_bytes / 2**20)
    order = [name for bucket in buckets for name in bucket.layout.parameter_names]
    assert order == [name for name, _ in reversed(params)]
    by_name = dict(params)

    def nbytes(name):
        p = by_name[name]
        return p.numel() * p.element_size()

    for index, bucket in enumerate(buckets):
        layout = bucket.layout
        assert layout.index == index
        members = [by_name[n] for n in layout.parameter_names]
        assert {p.dtype for p in members} == {members[0].dtype}
        assert layout.dtype_str == str(members[0].dtype)
        assert list(layout.numels) == [p.numel() for p in members]
        cursor = 0
        for offset, numel in zip(layout.offsets, layout.numels):
            assert offset == cursor
            cursor += numel
        assert layout.total_numel == cursor
        size = sum(nbytes(n) for n in layout.parameter_names)
        assert len(members) == 1 or size <= cap_bytes
        if index + 1 < len(buckets):
            following = buckets[index + 1].layout.parameter_names[0]
            if by_name[following].dtype == members[0].dtype:
                assert size + nbytes(following) > cap_bytes
        assert not bucket.is_allocated


@PROPERTY
@given(rows=st.lists(st.tuples(st.integers(0, 1 << 20), st.integers(0, 1 << 20), st.integers(0, 3000)),
                     max_size=8),
       chunk=st.sampled_from([256, 512]),
       scale=st.sampled_from([1, 2]))
def test_copy_table_assigns_every_chunk_to_the_row_that_holds_it(rows, chunk, scale):
    """The copy kernel finds chunk c's record as the last one whose ``first_chunk`` is
    at most c (zero-length rows share the next row's ``first_chunk`` and so own none).
    Enumerating every row's chunks must give the same owner and position."""
    flat, total = plan_table(rows, chunk, scale)
    records = [flat[4 * i:4 * i + 4] for i in range(len(rows))]
    assert [r[:3] for r in records] == [[s, d, n * scale] for s, d, n in rows]
    owners = []
    for index, (_, _, n) in enumerate(rows):
        k = 0
        while k * chunk < n * scale:
            owners.append((index, k))
            k += 1
    assert total == len(owners)
    firsts = [r[3] for r in records]
    for c, (index, k) in enumerate(owners):
        found = bisect.bisect_right(firsts, c) - 1
        assert (found, c - firsts[found]) == (index, k)


@PROPERTY
@given(sizes=st.lists(st.integers(0, 200_000), min_size=1, max_size=40), chunk=st.sampled_from([128, 256, 512]))
def test_copy_hints_name_the_record_of_every_256th_chunk(sizes, chunk):
    """``HBT_COPY_HINTS``: hint j is the owner of chunk 256 * j, found by brute force
    over every row's chunks; stepping forward from a chunk's hint while the next record
    starts at or before it lands on its owner (the kernel's search)."""
    rows = [(4096, 8192, n) for n in sizes]
    flat, total = plan_table(rows, chunk)
    hints = plan_hints(flat[3::4], total)
    owner = [i for i, (_, _, n) in enumerate(rows) for _ in range(-(-n // chunk))]
    assert len(owner) == total and len(hints) == -(-total // 256)
    assert hints == owner[::256]
    firsts = flat[3::4]
    for c in range(0, total, 97):
        r = hints[c >> 8]
        while r + 1 < len(rows) and firsts[r + 1] <= c:
            r += 1
        assert r == owner[c]


@PROPERTY
@given(numels=st.lists(st.integers(1, 40), min_size=1, max_size=6), writers=st.integers(1, 5), data=st.data())
def test_flat_sharded_manifest_round_trips_and_validates(numels, writers, data):
    """``checkpoint/manifest.py:63-561``: the manifest of a flat-sharded save, built
    piece by piece as writers record them, covers every element of every tensor once,
    survives its JSON form unchanged and validates.  Dropping a shard, a file's
    integrity record or the completion mark is refused with the reference's classes."""
    entries, total = build_flat_layout([(f"t{i}", torch.empty(n)) for i, n in enumerate(numels)])
    manifest = CheckpointManifest(writer_world_size=writers, step=7, complete=True)
    for rank, shard in enumerate(even_shard_ranges(total, writers)):
        name = shard_filename(rank)
        manifest.files[name] = FileRecord(name=name, sha256="0" * 64, bytes=1)
        for entry in entries:
            overlap = intersect_ranges(shard, ShardRange(entry.offset, entry.numel))
            if overlap is None:
                continue
            manifest.add_shard(
                TensorRecord(key=entry.name, name=entry.name, global_shape=entry.shape, dtype="torch.float32"),
                ShardRecord(rank=rank, file=name, offset=overlap.start - entry.offset, length=overlap.length,
                            key=entry.name),
            )
    for entry in entries:
        count = np.zeros(entry.numel, dtype=np.int64)
        for shard in manifest.tensors[entry.name].shards:
            count[shard.offset:shard.offset + shard.length] += 1
        assert (count == 1).all()
    manifest.validate()
    again = CheckpointManifest.from_dict(json.loads(manifest.to_json()))
    assert again.as_dict() == manifest.as_dict()
    again.validate()

    key = data.draw(st.sampled_from(sorted(again.tensors)), label="tensor")
    shards = again.tensors[key].shards
    del shards[data.draw(st.integers(0, len(shards) - 1), label="dropped shard")]
    with pytest.raises(IncompleteCheckpointError, match="do not cover"):
        again.validate()
    unrecorded = CheckpointManifest.from_dict(manifest.as_dict())
    unrecorded.files.pop(shard_filename(0))  # writer 0 always holds the first element
    with pytest.raises(IncompleteCheckpointError, match="integrity record"):
        unrecorded.validate()
    unfinished = CheckpointManifest.from_dict(manifest.as_dict())
    unfinished.complete = False
    with pytest.raises(IncompleteCheckpointError, match="not marked complete"):
        unfinished.validate()


@settings(deadline=None)
@given(total=st.integers(0, 2_000_000), chunk=st.integers(256, 1 << 22))
def test_host_stream_chunks_tile_the_pass_once(total, chunk):
    """The chunks of a streamed pass over host tensors cover [0, total) once, in order,
    each at most ``chunk`` long, only the last one shorter; and the norm pass's staged
    chunks, a whole number of norm chunks, keep every norm partial inside one chunk."""
    from hybrid_training_amd.host_staging import chunk_plan
    from hybrid_training_amd.optim import norm_chunk_elems

    plan = chunk_plan(total, chunk)
    assert sum(n for _, n in plan) == total
    cursor = 0
    for i, (start, n) in enumerate(plan):
        assert start == cursor and 0 < n <= chunk and (n == chunk or i == len(plan) - 1)
        cursor += n
    for dtype in (torch.float32, torch.bfloat16):
        nc = norm_chunk_elems(dtype)
        step = max(nc, chunk // nc * nc)  # the norm pass's staged chunk
        for start, n in chunk_plan(total, step):
            assert start % nc == 0  # the chunk's partials start at partial start // nc
    with pytest.raises(ValueError):
        chunk_plan(10, 0)
