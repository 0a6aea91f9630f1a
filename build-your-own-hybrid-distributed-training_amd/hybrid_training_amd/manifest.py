"""Checkpoint shard records: which file holds which interval of which tensor.

``ShardRecord`` and ``TensorRecord`` keep the fields, validation and JSON form of
``checkpoint/manifest.py:63-281`` of the reference, and ``validate_shard_filename``
enforces the same ``rank-NNNNN.pt`` naming rule (``checkpoint/format.py:80``,
``:176-205``), so records written by the reference load here.  The manifest file
itself (JSON I/O, file integrity records) is not part of this path.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field
from typing import Any

from .errors import CheckpointCorruptionError, CheckpointError, IncompleteCheckpointError, format_error
from .tensors import ShardRange, intersect_ranges

__all__ = ["ShardRecord", "TensorRecord", "shard_filename", "validate_shard_filename"]

_SHARD_FILENAME = re.compile(r"^rank-(\d{5,})\.pt$")


def shard_filename(rank: int) -> str:
    """``rank-NNNNN.pt`` for a writer rank (``checkpoint/format.py:139-162``)."""
    if rank < 0:
        raise CheckpointError(
            format_error("checkpoint.shard_filename", "rank must be non-negative", expected=">= 0",
                         observed=rank, resolution="pass a global rank")
        )
    return f"rank-{rank:05d}.pt"


def validate_shard_filename(name: str) -> str:
    """Reject anything but ``rank-NNNNN.pt`` (a manifest must not steer reads elsewhere)."""
    if not _SHARD_FILENAME.match(name):
        raise CheckpointError(
            format_error(
                "checkpoint.validate_shard_filename",
                "the manifest names a file that does not match the shard naming rule; "
                "refusing to read it, because a manifest must never be able to point "
                "the reader at an arbitrary path",
                expected="rank-NNNNN.pt",
                observed=name,
                resolution="the checkpoint directory has been tampered with or corrupted",
            )
        )
    return name


@dataclass(frozen=True)
class ShardRecord:
    """One contiguous piece of a global tensor (``manifest.py:63-125``)."""

    rank: int
    file: str
    offset: int
    length: int
    key: str
    padding: int = 0

    def __post_init__(self) -> None:
        if self.offset < 0 or self.length < 0:
            raise CheckpointError(
                format_error(
                    "manifest.ShardRecord",
                    "offset and length must be non-negative",
                    expected="offset >= 0 and length >= 0",
                    observed=f"offset={self.offset}, length={self.length}",
                    resolution="the manifest is malformed",
                )
            )
        validate_shard_filename(self.file)

    @property
    def range(self) -> ShardRange:
        """The interval this shard covers."""
        return ShardRange(start=self.offset, length=self.length)

    def as_dict(self) -> dict[str, Any]:
        """JSON form."""
        return {"rank": self.rank, "file": self.file, "offset": self.offset, "length": self.length,
                "key": self.key, "padding": self.padding}

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> ShardRecord:
        """Rebuild from :meth:`as_dict` output."""
        return cls(rank=int(payload["rank"]), file=str(payload["file"]), offset=int(payload["offset"]),
                   length=int(payload["length"]), key=str(payload["key"]),
                   padding=int(payload.get("padding", 0)))


@dataclass
class TensorRecord:
    """A global tensor and the shards that cover it (``manifest.py:128-281``)."""

    key: str
    name: str
    global_shape: tuple[int, ...]
    dtype: str
    category: str = "model"
    partition_dim: int | None = None
    tensor_parallel_size: int = 1
    tensor_parallel_rank: int = 0
    state_name: str = ""
    shards: list[ShardRecord] = field(default_factory=list)

    @property
    def numel(self) -> int:
        """Elements in the global tensor."""
        total = 1
        for dim in self.global_shape:
            total *= dim
        return total

    def covered_elements(self) -> int:
        """Distinct elements the shards cover (a union, so overlaps count once)."""
        if not self.shards:
            return 0
        covered, lo, hi = 0, None, None
        for start, end in sorted((s.offset, s.offset + s.length) for s in self.shards):
            if hi is None:
                lo, hi = start, end
            elif start > hi:
                covered += hi - lo
                lo, hi = start, end
            elif end > hi:
                hi = end
        return covered + (hi - lo)

    def validate(self) -> None:
        """The shards must tile the tensor exactly (``manifest.py:186-229``)."""
        for shard in self.shards:
            if shard.offset + shard.length > self.numel:
                raise CheckpointCorruptionError(
                    format_error(
                        "manifest.TensorRecord.validate",
                        f"a shard of {self.key!r} runs past the end of the tensor",
                        expected=f"offset + length <= {self.numel}",
                        observed=shard.offset + shard.length,
                        resolution="the manifest disagrees with the recorded global shape",
                    )
                )
        total = sum(s.length for s in self.shards)
        covered = self.covered_elements()
        if total != covered:
            raise CheckpointCorruptionError(
                format_error(
                    "manifest.TensorRecord.validate",
                    f"the shards of {self.key!r} overlap, so two files claim the same "
                    "elements and the reader cannot tell which is authoritative",
                    expected=f"{covered} elements across non-overlapping shards",
                    observed=total,
                    resolution="the checkpoint was written by a buggy or mixed-version writer",
                )
            )
        if covered != self.numel:
            raise IncompleteCheckpointError(
                format_error(
                    "manifest.TensorRecord.validate",
                    f"the shards of {self.key!r} do not cover the whole tensor",
                    expected=f"{self.numel} elements",
                    observed=covered,
                    resolution="a shard file is missing; the checkpoint is unusable",
                )
            )

    def shards_overlapping(self, wanted: ShardRange) -> list[tuple[ShardRecord, ShardRange]]:
        """``(shard, overlap)`` for every shard meeting ``wanted``, by offset (``:231-247``)."""
        out: list[tuple[ShardRecord, ShardRange]] = []
        for shard in sorted(self.shards, key=lambda s: s.offset):
            overlap = intersect_ranges(shard.range, wanted)
            if overlap is not None:
                out.append((shard, overlap))
        return out

    def as_dict(self) -> dict[str, Any]:
        """JSON form."""
        return {
            "key": self.key,
            "name": self.name,
            "global_shape": list(self.global_shape),
            "numel": self.numel,
            "dtype": self.dtype,
            "category": self.category,
            "partition_dim": self.partition_dim,
            "tensor_parallel_size": self.tensor_parallel_size,
            "tensor_parallel_rank": self.tensor_parallel_rank,
            "state_name": self.state_name,
            "shards": [s.as_dict() for s in sorted(self.shards, key=lambda s: s.offset)],
        }

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> TensorRecord:
        """Rebuild from :meth:`as_dict` output."""
        return cls(
            key=str(payload["key"]),
            name=str(payload["name"]),
            global_shape=tuple(int(d) for d in payload["global_shape"]),
            dtype=str(payload["dtype"]),
            category=str(payload.get("category", "model")),
            partition_dim=None if payload.get("partition_dim") is None else int(payload["partition_dim"]),
            tensor_parallel_size=int(payload.get("tensor_parallel_size", 1)),
            tensor_parallel_rank=int(payload.get("tensor_parallel_rank", 0)),
            state_name=str(payload.get("state_name", "")),
            shards=[ShardRecord.from_dict(s) for s in payload.get("shards", [])],
        )
