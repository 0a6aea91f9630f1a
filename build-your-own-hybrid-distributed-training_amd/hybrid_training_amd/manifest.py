"""The checkpoint format: manifest, shard records, file integrity, naming rules.

``ShardRecord``, ``TensorRecord``, ``FileRecord`` and ``CheckpointManifest`` keep the
fields, validation, errors and JSON form of ``checkpoint/manifest.py`` of the
reference, and the naming and path rules are those of ``checkpoint/format.py``
(``rank-NNNNN.pt`` payloads, ``manifest.json`` written last, staging directories,
format version "1.0"), so a checkpoint written by either side reads on the other.
"""

from __future__ import annotations

import hashlib
import json
import re
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

from .errors import (
    CheckpointCorruptionError,
    CheckpointError,
    CheckpointVersionError,
    IncompleteCheckpointError,
    format_error,
)
from .tensors import ShardRange, intersect_ranges

__all__ = [
    "CURRENT_FORMAT_VERSION",
    "CheckpointManifest",
    "FileRecord",
    "MANIFEST_FILENAME",
    "METADATA_FILENAME",
    "ShardRecord",
    "TensorRecord",
    "checkpoint_directory_name",
    "file_digest",
    "resolve_inside",
    "shard_filename",
    "staging_directory_name",
    "step_from_directory_name",
    "validate_format_version",
    "validate_shard_filename",
]

_SHARD_FILENAME = re.compile(r"^rank-(\d{5,})\.pt$")
CHECKPOINT_DIRECTORY_PATTERN = re.compile(r"^checkpoint-step-(\d{6,})$")
CURRENT_FORMAT_VERSION = "1.0"
SUPPORTED_FORMAT_VERSIONS = frozenset({"1.0"})
MANIFEST_FILENAME = "manifest.json"
METADATA_FILENAME = "metadata.json"
_STAGING_PREFIX = ".staging-"


def checkpoint_directory_name(step: int) -> str:
    """``checkpoint-step-NNNNNN`` (``checkpoint/format.py:85-108``)."""
    if step < 0:
        raise CheckpointError(
            format_error("checkpoint.directory_name", "step must be non-negative", expected=">= 0",
                         observed=step, resolution="pass the current optimizer step")
        )
    return f"checkpoint-step-{step:06d}"


def step_from_directory_name(name: str) -> int | None:
    """The step of a checkpoint directory name, or ``None``."""
    match = CHECKPOINT_DIRECTORY_PATTERN.match(name)
    return int(match.group(1)) if match else None


def staging_directory_name(final_name: str, token: str) -> str:
    """The hidden directory a checkpoint is written into before its atomic rename."""
    return f"{_STAGING_PREFIX}{final_name}-{token}"


def validate_format_version(version: str) -> str:
    """Refuse a format version this library cannot read."""
    if version not in SUPPORTED_FORMAT_VERSIONS:
        raise CheckpointVersionError(
            format_error(
                "checkpoint.validate_format_version",
                "the checkpoint was written in a format version this library cannot read",
                expected=sorted(SUPPORTED_FORMAT_VERSIONS),
                observed=version,
                resolution="read it with the version of the package that wrote it",
            )
        )
    return version


def resolve_inside(root: Path, name: str) -> Path:
    """``root / name``, proven to stay inside ``root`` after resolving symlinks."""
    root_resolved = Path(root).resolve()
    candidate = (root_resolved / name).resolve()
    try:
        candidate.relative_to(root_resolved)
    except ValueError as exc:
        raise CheckpointError(
            format_error(
                "checkpoint.resolve_inside",
                "the resolved path escapes the checkpoint directory",
                expected=f"a path under {root_resolved}",
                observed=str(candidate),
                resolution="remove the symlink or path component that redirects outside",
            )
        ) from exc
    return candidate


def file_digest(path: Path, *, chunk_size: int = 1 << 22) -> str:
    """SHA-256 hex digest of a file, streamed in chunks."""
    digest = hashlib.sha256()
    with open(path, "rb") as handle:
        while True:
            block = handle.read(chunk_size)
            if not block:
                break
            digest.update(block)
    return digest.hexdigest()


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


@dataclass(frozen=True)
class FileRecord:
    """Integrity metadata of one payload file (``checkpoint/manifest.py:286-311``)."""

    name: str
    sha256: str
    bytes: int

    def as_dict(self) -> dict[str, Any]:
        """JSON form."""
        return {"name": self.name, "sha256": self.sha256, "bytes": self.bytes}

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> FileRecord:
        """Rebuild from :meth:`as_dict` output."""
        return cls(name=validate_shard_filename(str(payload["name"])), sha256=str(payload["sha256"]),
                   bytes=int(payload["bytes"]))


@dataclass
class CheckpointManifest:
    """The rank-independent description of a checkpoint (``checkpoint/manifest.py:314-561``)."""

    format_version: str = CURRENT_FORMAT_VERSION
    writer_world_size: int = 1
    topology: dict[str, Any] = field(default_factory=dict)
    step: int = 0
    tensors: dict[str, TensorRecord] = field(default_factory=dict)
    files: dict[str, FileRecord] = field(default_factory=dict)
    complete: bool = False
    created_by: str = ""

    def add_shard(self, record: TensorRecord, shard: ShardRecord) -> None:
        """Register one shard, creating or extending the tensor's record."""
        existing = self.tensors.get(record.key)
        if existing is None:
            self.tensors[record.key] = TensorRecord(
                key=record.key, name=record.name, global_shape=record.global_shape, dtype=record.dtype,
                category=record.category, partition_dim=record.partition_dim,
                tensor_parallel_size=record.tensor_parallel_size,
                tensor_parallel_rank=record.tensor_parallel_rank, state_name=record.state_name,
                shards=[shard],
            )
            return
        if existing.global_shape != record.global_shape or existing.dtype != record.dtype:
            raise CheckpointCorruptionError(
                format_error(
                    "manifest.add_shard",
                    f"two ranks describe tensor {record.key!r} differently, so the "
                    "manifest cannot describe a single global tensor",
                    expected=f"shape={existing.global_shape}, dtype={existing.dtype}",
                    observed=f"shape={record.global_shape}, dtype={record.dtype}",
                    resolution=(
                        "the ranks are running different model definitions; check that "
                        "every rank built the model from the same configuration"
                    ),
                )
            )
        existing.shards.append(shard)

    def validate(self) -> None:
        """Complete, version-readable, every tensor tiled, every file recorded."""
        validate_format_version(self.format_version)
        if not self.complete:
            raise IncompleteCheckpointError(
                format_error(
                    "manifest.validate",
                    "the manifest is not marked complete, which means the writer did not "
                    "finish; a checkpoint is only published after every shard validates",
                    expected=True,
                    observed=self.complete,
                    resolution="discard this checkpoint and resume from an earlier one",
                )
            )
        for record in self.tensors.values():
            record.validate()
            for shard in record.shards:
                if shard.file not in self.files:
                    raise IncompleteCheckpointError(
                        format_error(
                            "manifest.validate",
                            f"tensor {record.key!r} references file {shard.file!r}, which "
                            "has no integrity record",
                            expected=sorted(self.files),
                            observed=shard.file,
                            resolution="the manifest is truncated or hand-edited",
                        )
                    )

    def referenced_files(self) -> set[str]:
        """File names any tensor depends on."""
        return {shard.file for record in self.tensors.values() for shard in record.shards}

    def tensors_by_category(self, category: str) -> dict[str, TensorRecord]:
        """The records of one category (``"model"``, ``"optimizer"``, ``"buffer"``)."""
        return {k: v for k, v in self.tensors.items() if v.category == category}

    def as_dict(self) -> dict[str, Any]:
        """JSON form with a deterministic key order."""
        return {
            "format_version": self.format_version,
            "created_by": self.created_by,
            "writer_world_size": self.writer_world_size,
            "topology": self.topology,
            "step": self.step,
            "complete": self.complete,
            "tensors": {k: self.tensors[k].as_dict() for k in sorted(self.tensors)},
            "files": {k: self.files[k].as_dict() for k in sorted(self.files)},
        }

    def to_json(self, *, indent: int | None = 2) -> str:
        """The manifest as JSON text."""
        return json.dumps(self.as_dict(), indent=indent, sort_keys=True)

    def write(self, path: Path) -> Path:
        """Write the manifest to ``path``."""
        Path(path).write_text(self.to_json(), encoding="utf-8")
        return Path(path)

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> CheckpointManifest:
        """Rebuild from :meth:`as_dict` output; a malformed payload raises ``CheckpointError``."""
        try:
            return cls(
                format_version=str(payload["format_version"]),
                created_by=str(payload.get("created_by", "")),
                writer_world_size=int(payload.get("writer_world_size", 1)),
                topology=dict(payload.get("topology", {})),
                step=int(payload.get("step", 0)),
                complete=bool(payload.get("complete", False)),
                tensors={k: TensorRecord.from_dict(v) for k, v in payload.get("tensors", {}).items()},
                files={k: FileRecord.from_dict(v) for k, v in payload.get("files", {}).items()},
            )
        except (KeyError, TypeError, ValueError) as exc:
            raise CheckpointError(
                format_error(
                    "manifest.from_dict",
                    "the manifest is malformed",
                    expected="a manifest written by this package",
                    observed=repr(exc),
                    resolution="the file is not a valid checkpoint manifest",
                )
            ) from exc

    @classmethod
    def read(cls, path: Path) -> CheckpointManifest:
        """Load (not yet validate) a manifest; a missing file means an unfinished write."""
        path = Path(path)
        if not path.is_file():
            raise IncompleteCheckpointError(
                format_error(
                    "manifest.read",
                    "no manifest found; the manifest is written last, so its absence "
                    "means the checkpoint was never completed",
                    expected=str(path),
                    observed="missing",
                    resolution="resume from an earlier checkpoint",
                )
            )
        try:
            payload = json.loads(path.read_text(encoding="utf-8"))
        except json.JSONDecodeError as exc:
            raise CheckpointError(
                format_error("manifest.read", "the manifest is not valid JSON", expected="a JSON object",
                             observed=str(exc), resolution="the file is corrupt")
            ) from exc
        if not isinstance(payload, dict):
            raise CheckpointError(
                format_error("manifest.read", "the manifest is not a JSON object", expected="object",
                             observed=type(payload).__name__, resolution="the file is corrupt")
            )
        return cls.from_dict(payload)
