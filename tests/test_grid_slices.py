"""How libhbt.so splits an oversized grid into launches (no GPU).

A HIP grid dimension holds at most 2^32 - 1 work-items (workgroups x workgroup size).
Every kernel launch in the library goes through one split, exported as
``hbt_grid_slices``: consecutive slices of at most floor((2^32 - 1) / threads)
workgroups.  The property below checks it against that definition on generated
sizes, and the known answers pin the sizes that matter: a Llama-3-70B fp32 unpack
(70,553,706,496 elements, 1 KB chunks of 64-lane workgroups) needs five launches,
and the headline AdamW shard one.  Checking ``blocks <= 2^31 - 1`` instead, as a
guard on the block count alone would, accepts grids of 64-lane workgroups 32 times
too large; the last test shows the difference.
"""

from __future__ import annotations

from hypothesis import given, settings
from hypothesis import strategies as st

from hybrid_training_amd import _native

MAX_ITEMS = 2**32 - 1


def _slices(blocks: int, threads: int) -> list[tuple[int, int]]:
    lib = _native.library()
    n = int(lib.hbt_grid_slices(blocks, threads, None, None, 0))
    first = _native.int64_array([0] * max(n, 1))
    count = _native.int64_array([0] * max(n, 1))
    assert lib.hbt_grid_slices(blocks, threads, first, count, n) == n
    return [(first[k], count[k]) for k in range(n)]


@settings(max_examples=200, derandomize=True, deadline=None)
@given(blocks=st.integers(min_value=0, max_value=2**40), threads=st.sampled_from([1, 32, 64, 256, 1000, 1024]))
def test_slices_tile_the_grid_within_the_work_item_limit(blocks, threads):
    slices = _slices(blocks, threads)
    per = MAX_ITEMS // threads
    assert len(slices) == -(-blocks // per)  # as few launches as the limit allows
    cursor = 0
    for first, count in slices:
        assert first == cursor and 0 < count <= per
        assert count * threads <= MAX_ITEMS
        cursor += count
    assert cursor == blocks


def test_known_answers():
    # fp32 unpack of Llama-3-70B: 1 KB (256-element) chunks, 64-lane workgroups
    chunks = -(-70_553_706_496 // 256)
    slices = _slices(chunks, 64)
    assert len(slices) == 5 and slices[0] == (0, 67_108_863) and slices[-1][0] == 4 * 67_108_863
    # the headline AdamW shard: 256 elements per 32-lane workgroup, one launch
    assert _slices(-(-1_003_782_656 // 256), 32) == [(0, 3_921_026)]
    # the Llama-3-70B rank shard's bf16 norm: 65,536 elements per 1024-lane workgroup
    assert _slices(-(-8_819_213_312 // 65536), 1024) == [(0, 134_571)]
    assert _slices(0, 64) == [] and _native.library().hbt_grid_slices(5, 0, None, None, 0) == -1


def test_a_block_count_guard_would_admit_oversized_grids():
    blocks = 2**31 - 1  # passes `blocks <= 0x7FFFFFFF`
    assert blocks * 64 > MAX_ITEMS
    assert len(_slices(blocks, 64)) == 33  # ceil((2^31 - 1) / floor((2^32 - 1) / 64))
