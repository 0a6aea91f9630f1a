"""Checkpoint resharding as device interval copies.

A checkpoint stores every tensor as shards: intervals of its row-major flattening.
A loading rank wants intervals of its own; the bytes to move are the
intersections, whatever the saving and loading widths were.  This module keeps the
reference's reader interface (``read_tensor_range``, ``checkpoint/reshard.py:200-305``)
and error behaviour, and adds :func:`load_flat_shard`, the FSDP destination fill of
``checkpoint/reader.py:328-351`` (and the optimizer-state fill of ``:423-443``) done
as ONE launch of the interval copy kernel straight from the stored shards into the
destination shard.  The reference copies twice per piece (into a temporary, then
into the destination) and runs a Python loop per piece.

Payloads are resident on the device: :class:`DeviceShardCache` holds tensors
already there, and ``checkpoint.ShardFileCache`` verifies, loads and uploads
``.pt`` files.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping, Sequence
from typing import Any

import torch

from . import _native
from .errors import CheckpointCorruptionError, CheckpointError, IncompleteCheckpointError, format_error
from .flat_param import PieceLayout
from .manifest import CheckpointManifest, TensorRecord, validate_shard_filename
from .tensors import ShardRange

__all__ = ["DeviceShardCache", "describe_reshard", "load_flat_shard", "read_tensor_range"]


class DeviceShardCache:
    """Shard payloads already on the device, keyed like ``ShardFileCache`` (``reshard.py:54-197``).

    ``payloads`` maps a shard file name (``rank-NNNNN.pt``) to ``{storage_key: tensor}``.
    """

    def __init__(self, payloads: Mapping[str, Mapping[str, torch.Tensor]] | None = None) -> None:
        self._payloads: dict[str, dict[str, torch.Tensor]] = {}
        self._loaded: set[str] = set()
        for name, payload in (payloads or {}).items():
            for key, tensor in payload.items():
                self.add(name, key, tensor)

    def add(self, filename: str, key: str, tensor: torch.Tensor) -> None:
        """Register one stored shard tensor."""
        validate_shard_filename(filename)
        _native.require_device_tensor(tensor, "reshard.DeviceShardCache")
        self._payloads.setdefault(filename, {})[key] = tensor

    def get(self, filename: str) -> Mapping[str, torch.Tensor]:
        """The tensors stored under ``filename``."""
        payload = self._payloads.get(validate_shard_filename(filename))
        if payload is None:
            raise IncompleteCheckpointError(
                format_error(
                    "reshard.DeviceShardCache.get",
                    f"payload {filename!r} is missing from the device cache",
                    observed=sorted(self._payloads)[:8],
                    resolution="add every payload file the manifest lists before reading",
                )
            )
        self._loaded.add(filename)
        return payload

    def loaded_files(self) -> tuple[str, ...]:
        """Files read so far."""
        return tuple(sorted(self._loaded))


def _queue_range(
    record: TensorRecord,
    wanted: ShardRange,
    cache: DeviceShardCache,
    dest: torch.Tensor | None,
    dest_offset: int,
    add: Callable[[torch.Tensor, int, int, int], None],
) -> torch.dtype:
    """Queue the copies that fill ``wanted`` of ``record``; returns the first shard's dtype.

    ``add(source_flat, source_offset, dest_offset, length)`` receives one interval per
    intersecting shard, in offset order.  The checks are those of ``reshard.py:224-302``,
    in the same order and with the same exception classes.
    """
    if wanted.end > record.numel:
        raise CheckpointError(
            format_error(
                "reshard.read_tensor_range",
                f"range [{wanted.start}, {wanted.end}) of {record.key!r} reaches past the end of "
                f"the saved tensor ({record.numel} elements)",
                observed=wanted.end,
                resolution="the model being loaded is larger than the one saved",
            )
        )
    overlaps = record.shards_overlapping(wanted)
    if not overlaps:
        raise IncompleteCheckpointError(
            format_error(
                "reshard.read_tensor_range",
                f"none of the saved intervals of {record.key!r} meets [{wanted.start}, {wanted.end})",
                observed=[(s.offset, s.length) for s in record.shards],
                resolution="the writer that held this interval left no record",
            )
        )
    first_dtype: torch.dtype | None = None
    filled = 0
    cursor = wanted.start
    for shard, overlap in overlaps:
        if overlap.start != cursor:
            raise IncompleteCheckpointError(
                format_error(
                    "reshard.read_tensor_range",
                    f"elements [{cursor}, {overlap.start}) of {record.key!r} are in no shard (a gap)",
                    resolution="the writer that held them left no record",
                )
            )
        payload = cache.get(shard.file)
        stored = payload.get(shard.key)
        if stored is None:
            raise CheckpointCorruptionError(
                format_error(
                    "reshard.read_tensor_range",
                    f"payload {shard.file!r} holds no entry {shard.key!r}",
                    observed=sorted(payload)[:8],
                    resolution="manifest and payload were not written together",
                )
            )
        flat = _native.contiguous_source(stored.reshape(-1))
        if flat.numel() != shard.length:
            raise CheckpointCorruptionError(
                format_error(
                    "reshard.read_tensor_range",
                    f"entry {shard.key!r} holds {flat.numel()} elements, its record says {shard.length}",
                    resolution="manifest and payload were not written together",
                )
            )
        if first_dtype is None:
            first_dtype = flat.dtype
        add(flat, overlap.start - shard.offset, dest_offset + filled, overlap.length)
        filled += overlap.length
        cursor = overlap.end
    if filled != wanted.length:
        raise IncompleteCheckpointError(
            format_error(
                "reshard.read_tensor_range",
                f"the shards of {record.key!r} supply {filled} of the {wanted.length} elements "
                f"of [{wanted.start}, {wanted.end})",
                resolution="the writer that held the rest left no record",
            )
        )
    assert first_dtype is not None
    return first_dtype


class _PlanSet:
    """Copy plans keyed by source dtype, all writing one destination dtype."""

    def __init__(self, device: torch.device, dst_dtype: torch.dtype) -> None:
        self.device = device
        self.dst_dtype = dst_dtype
        self.plans: dict[torch.dtype, _native.CopyPlan] = {}

    def add(self, src: torch.Tensor, src_offset: int, dst: torch.Tensor, dst_offset: int, n: int) -> None:
        if src.dtype != dst.dtype and (src.dtype, dst.dtype) not in _native.COPY_CONVERSIONS:
            raise CheckpointError(
                format_error("reshard.read_tensor_range", "unsupported dtype conversion",
                             observed=f"{src.dtype} -> {dst.dtype}")
            )
        self.plans.setdefault(src.dtype, _native.CopyPlan(self.device)).add(src, src_offset, dst, dst_offset, n)

    def run(self) -> None:
        for src_dtype, plan in self.plans.items():
            plan.run(src_dtype=src_dtype, dst_dtype=self.dst_dtype)


def read_tensor_range(
    record: TensorRecord,
    wanted: ShardRange,
    cache: DeviceShardCache,
    *,
    dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Elements ``wanted`` of a stored tensor as a new 1-D device tensor (one launch).

    ``dtype`` casts the result as ``Tensor.to`` does (``checkpoint/reshard.py:290``), between any
    of float64, float32, bfloat16 and float16; by default the result has the first
    intersecting shard's dtype.
    """
    if wanted.length == 0:
        device = next(
            (t.device for name in (s.file for s in record.shards) for t in cache.get(name).values()),
            None,
        )
        return torch.empty(0, dtype=dtype or torch.float32, device=device)
    pending: list[tuple[torch.Tensor, int, int, int]] = []
    first = _queue_range(record, wanted, cache, None, 0,
                         lambda src, so, do, n: pending.append((src, so, do, n)))
    out_dtype = dtype or first
    out = torch.empty(wanted.length, dtype=out_dtype, device=pending[0][0].device)
    plans = _PlanSet(out.device, out_dtype)
    for src, so, do, n in pending:
        plans.add(src, so, out, do, n)
    plans.run()
    return out


def load_flat_shard(
    destination: torch.Tensor,
    layout: Sequence[PieceLayout],
    records: Mapping[str, TensorRecord],
    cache: DeviceShardCache,
    *,
    key_of: Callable[[PieceLayout], str] | None = None,
    strict: bool = True,
) -> int:
    """Fill a flat shard's pieces from the checkpoint in one launch; returns pieces loaded.

    ``layout`` is the destination's ``local_piece_layout()`` (``fsdp.py:810-843``);
    each piece ``(name, parameter_offset, length, local_offset)`` receives elements
    ``[parameter_offset, parameter_offset + length)`` of the stored tensor at
    ``destination[local_offset:]``, cast to the destination dtype.  ``key_of`` maps
    a piece to its record key (default: the piece name; optimizer state uses
    ``f"{name}::{state}"``).  A missing record raises ``IncompleteCheckpointError``
    when ``strict``, else the piece is left unchanged (``reader.py:328-351``).
    """
    _native.require_device_tensor(destination, "reshard.load_flat_shard")
    dest = destination.detach().view(-1)
    if not dest.is_contiguous():
        raise CheckpointError(format_error("reshard.load_flat_shard", "the destination must be dense"))
    plans = _PlanSet(dest.device, dest.dtype)
    loaded = 0
    for item in layout:
        key = key_of(item) if key_of is not None else item.name
        record = records.get(key)
        if record is None:
            if strict:
                raise IncompleteCheckpointError(
                    format_error(
                        "checkpoint.load",
                        f"the checkpoint has no tensor {key!r}",
                        expected=key,
                        observed=sorted(records)[:8],
                        resolution="load a checkpoint produced by the same model definition",
                    )
                )
            continue
        if item.local_offset + item.length > dest.numel():
            raise CheckpointError(
                format_error("reshard.load_flat_shard", "a piece runs past the destination shard",
                             expected=f"<= {dest.numel()}", observed=item.local_offset + item.length)
            )
        if item.length == 0:
            continue
        _queue_range(record, ShardRange(item.parameter_offset, item.length), cache, dest,
                     item.local_offset,
                     lambda src, so, do, n: plans.add(src, so, dest, do, n))
        loaded += 1
    plans.run()
    return loaded


def describe_reshard(manifest: CheckpointManifest, key: str, wanted: ShardRange) -> dict[str, Any]:
    """The plan of a read, without reading (``reshard.py:377-421``): which saved shards
    the interval ``wanted`` of tensor ``key`` touches, and where."""
    record = manifest.tensors.get(key)
    if record is None:
        raise CheckpointError(
            format_error(
                "reshard.describe_reshard",
                f"unknown tensor key {key!r}",
                observed=sorted(manifest.tensors)[:8],
                resolution="use a key listed in the manifest's tensors",
            )
        )
    return {
        "key": key,
        "global_shape": list(record.global_shape),
        "wanted": [wanted.start, wanted.length],
        "sources": [
            {"file": shard.file, "saved_rank": shard.rank, "shard_range": [shard.offset, shard.length],
             "overlap": [overlap.start, overlap.length]}
            for shard, overlap in record.shards_overlapping(wanted)
        ],
    }
