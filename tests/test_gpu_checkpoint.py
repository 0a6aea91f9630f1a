"""Save a sharded model and its AdamW state to disk, load it back at other widths.

Reference behaviour (``tests/integration/test_checkpoint.py:331-412``): an FSDP
checkpoint saved at one shard-group width restores bitwise at another, and the
optimizer state follows its parameters.  Here four writers save a 270,310-element
model (shards padded by 2) after two AdamW steps; readers at W = 4, 3, 8 and 1 load
it with ``load_flat_shard_checkpoint``.  Every loaded shard and state tensor must
equal the corresponding slice of the global flat vectors bitwise, and the step
counter must come back; a corrupted file must be refused.
"""

from __future__ import annotations

import pytest
import torch

from hybrid_training_amd import (
    CheckpointManifest,
    FlatParamHandle,
    FSDPConfig,
    GroupHandle,
    MixedPrecisionConfig,
    OptimizerConfig,
    ShardedOptimizer,
    ShardFileCache,
    collect_flat_shard_payload,
    load_flat_shard_checkpoint,
    write_checkpoint,
)
from hybrid_training_amd.errors import CheckpointCorruptionError
from hybrid_training_amd.manifest import MANIFEST_FILENAME

pytestmark = pytest.mark.gpu

SHAPES = [("a", (700, 300)), ("b", (301,)), ("c", (200, 300)), ("d", (9,))]
TOTAL = 270_310


def _model(device, seed=9):
    gen = torch.Generator(device=device).manual_seed(seed)
    return [(n, torch.nn.Parameter(torch.randn(s, device=device, generator=gen))) for n, s in SHAPES]


def _world(named, group, device):
    handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r), FSDPConfig(),
                               MixedPrecisionConfig(), device, keep_originals=True) for r in range(group)]
    opts = [ShardedOptimizer([h.flat_param], OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                             norm_group=GroupHandle.local_view("world", group, r), device=device)
            for r, h in enumerate(handles)]
    return handles, opts


def _global(shards, total):
    return torch.cat([s.detach().reshape(-1) for s in shards])[:total]


@pytest.fixture
def saved(tmp_path, device):
    named = _model(device)
    handles, opts = _world(named, 4, device)
    gen = torch.Generator(device=device).manual_seed(1)
    for _ in range(2):
        for h, opt in zip(handles, opts):
            h.flat_param.grad = torch.randn(h.shard_numel, device=device, generator=gen) * 1e-2
            opt.step()
    shards = [(r, *collect_flat_shard_payload(h, rank=r, optimizer=opt)) for r, (h, opt) in
              enumerate(zip(handles, opts))]
    path = write_checkpoint(tmp_path, 2, shards, topology={"fsdp": 4})
    flat = _global([h.flat_param for h in handles], TOTAL)
    m = _global([o.inner.state[h.flat_param]["exp_avg"] for h, o in zip(handles, opts)], TOTAL)
    v = _global([o.inner.state[h.flat_param]["exp_avg_sq"] for h, o in zip(handles, opts)], TOTAL)
    return path, flat, m, v


@pytest.mark.parametrize("group", [4, 3, 8, 1])
def test_load_at_any_width(device, saved, group):
    path, flat, m, v = saved
    named = _model(device, seed=123)  # different initial values: everything must come from disk
    handles, opts = _world(named, group, device)
    writer_shard = -(-TOTAL // 4)
    for r, (h, opt) in enumerate(zip(handles, opts)):
        cache = ShardFileCache(path, CheckpointManifest.read(path / MANIFEST_FILENAME), device=device)
        loaded = load_flat_shard_checkpoint(path, h, optimizer=opt, cache=cache)
        assert loaded == len(h.local_piece_layout())
        # a reader opens exactly the writers' files its interval intersects (tests/integration/
        # test_checkpoint.py:351-371; the reference's extra file holds RNG state, not on this path)
        lo, hi = r * h.shard_numel, min(TOTAL, (r + 1) * h.shard_numel)
        expect = {f"rank-{k:05d}.pt" for k in range(4) if k * writer_shard < hi and lo < (k + 1) * writer_shard}
        assert set(cache.loaded_files) == expect, (r, cache.loaded_files)
        start = r * h.shard_numel
        valid = max(0, min(h.shard_numel, TOTAL - start))
        assert torch.equal(h.flat_param.detach()[:valid], flat[start : start + valid])
        assert float(h.flat_param.detach()[valid:].abs().sum()) == 0.0  # padding stays zero
        state = opt.inner.state[h.flat_param]
        assert torch.equal(state["exp_avg"][:valid], m[start : start + valid])
        assert torch.equal(state["exp_avg_sq"][:valid], v[start : start + valid])
        assert float(state["step"]) == 2.0


def test_corrupt_payload_is_refused(device, saved):
    path, *_ = saved
    target = path / "rank-00002.pt"
    raw = bytearray(target.read_bytes())
    raw[-100] ^= 0x01
    target.write_bytes(bytes(raw))
    named = _model(device)
    handles, opts = _world(named, 2, device)
    with pytest.raises(CheckpointCorruptionError, match="checksum"):
        load_flat_shard_checkpoint(path, handles[1], optimizer=opts[1])


def test_padding_only_ranks_save_and_load_optimizer_state(device, tmp_path):
    """A one-element model saved by 3 writers and loaded by 4 readers: every rank but the
    first owns padding only, so it has no piece to write or read.  Its load still
    succeeds, strict, with zero moments and the saved step; rank 0 gets the saved values."""
    named = [("w", torch.nn.Parameter(torch.full((1,), 0.5, device=device)))]
    handles, opts = _world(named, 3, device)
    for h, opt in zip(handles, opts):
        h.flat_param.grad = torch.full((h.shard_numel,), 0.25, device=device)
        opt.step()
    payloads = [(r, *collect_flat_shard_payload(h, rank=r, optimizer=o)) for r, (h, o) in
                enumerate(zip(handles, opts))]
    path = write_checkpoint(tmp_path, 1, payloads, topology={"fsdp": 3})
    saved_p = handles[0].flat_param.detach()[:1].clone()
    saved_m = opts[0].inner.state[handles[0].flat_param]["exp_avg"][:1].clone()
    readers, reader_opts = _world([("w", torch.nn.Parameter(torch.zeros(1, device=device)))], 4, device)
    for r, (h, o) in enumerate(zip(readers, reader_opts)):
        load_flat_shard_checkpoint(path, h, optimizer=o)
        state = o.inner.state[h.flat_param]
        assert float(state["step"]) == 1.0, r
        if r == 0:
            assert torch.equal(h.flat_param.detach()[:1], saved_p) and torch.equal(state["exp_avg"][:1], saved_m)
        else:
            assert float(state["exp_avg"].abs().sum()) == 0.0 and float(state["exp_avg_sq"].abs().sum()) == 0.0
            assert float(h.flat_param.detach().abs().sum()) == 0.0
