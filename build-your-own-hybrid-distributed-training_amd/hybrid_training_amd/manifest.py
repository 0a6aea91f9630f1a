"""Checkpoint records, and the naming, path and integrity rules of a checkpoint directory.

A checkpoint is a directory ``checkpoint-step-NNNNNN/`` holding one ``rank-NNNNN.pt``
payload per writer, ``metadata.json``, and ``manifest.json``, which says which global
interval of which tensor each payload key carries, plus every payload's SHA-256 and
size.  The manifest is written last, so a directory without one is unfinished.

What has to match the reference for checkpoints to move between the two is kept as
data: the record classes and their fields, the JSON keys (``checkpoint/manifest.py:63-561``),
the file and directory name rules and the format version "1.0"
(``checkpoint/format.py:59-292``), and the exception classes.  Error messages are this
package's own; each keeps the short phrase the reference's tests match
(``tests/unit/test_checkpoint_format.py:59-313``,
``tests/integration/test_checkpoint.py:461-522``), so handlers keyed on those phrases work.
"""

from __future__ import annotations

import hashlib
import json
import re
from dataclasses import dataclass, field, fields
from pathlib import Path
from typing import Any, Callable, NoReturn

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

CURRENT_FORMAT_VERSION = "1.0"
SUPPORTED_FORMAT_VERSIONS = frozenset({CURRENT_FORMAT_VERSION})
MANIFEST_FILENAME = "manifest.json"
METADATA_FILENAME = "metadata.json"
# Name rules (checkpoint/format.py:72-80): at least six step digits, five rank digits.
CHECKPOINT_DIRECTORY_PATTERN = re.compile(r"^checkpoint-step-(\d{6,})$")
_PAYLOAD_NAME = re.compile(r"^rank-(\d{5,})\.pt$")
_STAGING_PREFIX = ".staging-"


def _fail(kind: type[Exception], where: str, problem: str, *, expected: Any = None, observed: Any = None,
          fix: str | None = None, cause: BaseException | None = None) -> NoReturn:
    """Raise ``kind`` with a ``format_error`` message (chained to ``cause`` when given)."""
    raise kind(format_error(where, problem, expected=expected, observed=observed, resolution=fix)) from cause


# ---- names and paths ------------------------------------------------------------------
def checkpoint_directory_name(step: int) -> str:
    """``checkpoint-step-NNNNNN`` for an optimizer step (``checkpoint/format.py:85-108``)."""
    if step < 0:
        _fail(CheckpointError, "checkpoint.directory_name", "step must be non-negative",
              observed=step, fix="name checkpoints by the optimizer step that produced them")
    return f"checkpoint-step-{step:06d}"


def step_from_directory_name(name: str) -> int | None:
    """The step encoded in a checkpoint directory name, or ``None`` for other names."""
    found = CHECKPOINT_DIRECTORY_PATTERN.fullmatch(name)
    return None if found is None else int(found.group(1))


def staging_directory_name(final_name: str, token: str) -> str:
    """Hidden sibling a checkpoint is assembled in before one rename publishes it."""
    return _STAGING_PREFIX + final_name + "-" + token


def shard_filename(rank: int) -> str:
    """``rank-NNNNN.pt``, the payload file of one writer (``checkpoint/format.py:139-162``)."""
    if rank < 0:
        _fail(CheckpointError, "checkpoint.shard_filename", "rank must be non-negative",
              observed=rank, fix="payload files are named after a global rank")
    return f"rank-{rank:05d}.pt"


def validate_shard_filename(name: str) -> str:
    """``name`` if it is a payload file name, else :class:`CheckpointError`.

    Every file name read from a manifest passes through here before it is joined to a
    directory, so manifest text alone cannot send a reader to another path.
    """
    if _PAYLOAD_NAME.fullmatch(name) is None:
        _fail(CheckpointError, "checkpoint.validate_shard_filename",
              "file name does not match the shard naming rule (rank-NNNNN.pt); it is not read",
              observed=name, fix="rebuild the manifest from the payload files the writers produced")
    return name


def resolve_inside(root: Path, name: str) -> Path:
    """``root / name`` with symlinks resolved, refused unless it still lies under ``root``."""
    base = Path(root).resolve()
    target = (base / name).resolve()
    if target != base and base not in target.parents:
        _fail(CheckpointError, "checkpoint.resolve_inside",
              "path escapes the checkpoint directory once links are resolved",
              expected=f"inside {base}", observed=str(target),
              fix="remove the link or '..' component that leads out of the directory")
    return target


def validate_format_version(version: str) -> str:
    """``version`` if this package reads it, else :class:`CheckpointVersionError`."""
    if version not in SUPPORTED_FORMAT_VERSIONS:
        _fail(CheckpointVersionError, "checkpoint.validate_format_version",
              "unsupported checkpoint format version", expected=sorted(SUPPORTED_FORMAT_VERSIONS),
              observed=version, fix="load it with the release that wrote it, or convert it first")
    return version


def file_digest(path: Path, *, chunk_size: int = 1 << 22) -> str:
    """Lowercase hex SHA-256 of a file, read in ``chunk_size`` pieces.

    An unreadable file (absent, a directory, no permission) raises
    :class:`CheckpointError`, not the ``OSError`` underneath (``checkpoint/format.py:246-262``).
    """
    hasher = hashlib.sha256()
    try:
        with open(path, "rb") as stream:
            for piece in iter(lambda: stream.read(chunk_size), b""):
                hasher.update(piece)
    except OSError as err:
        _fail(CheckpointError, "checkpoint.file_digest", "could not read a checkpoint file",
              observed=f"{path} ({err.__class__.__name__}: {err.strerror or err})",
              fix="make sure the file exists and is readable", cause=err)
    return hasher.hexdigest()


# ---- JSON codec -------------------------------------------------------------------------
_REQUIRED = object()


def _decode(payload: dict[str, Any], spec: tuple[tuple[str, Callable[[Any], Any], Any], ...]) -> dict[str, Any]:
    """Constructor arguments from a JSON object: ``(key, convert, default)`` per field,
    ``default`` (converted like a stored value) or ``_REQUIRED`` for keys that must be present.  A missing key or a
    value ``convert`` rejects raises ``KeyError`` / ``TypeError`` / ``ValueError``."""
    out: dict[str, Any] = {}
    for key, convert, default in spec:
        if key in payload:
            out[key] = convert(payload[key])
        elif default is _REQUIRED:
            raise KeyError(key)
        else:
            out[key] = convert(default)  # a fresh value each time (dict({}) is a new dict)
    return out


def _optional_int(value: Any) -> int | None:
    return None if value is None else int(value)


def _int_tuple(value: Any) -> tuple[int, ...]:
    return tuple(int(v) for v in value)


def _by_offset(shards: list[ShardRecord]) -> list[ShardRecord]:
    return sorted(shards, key=lambda s: s.offset)


# ---- records ---------------------------------------------------------------------------
@dataclass(frozen=True)
class ShardRecord:
    """Elements ``[offset, offset + length)`` of a tensor's row-major flattening, stored
    under ``key`` in payload ``file`` by writer ``rank``; the last ``padding`` of them
    are flat-parameter padding (``checkpoint/manifest.py:63-125``)."""

    rank: int
    file: str
    offset: int
    length: int
    key: str
    padding: int = 0

    _SPEC = (("rank", int, _REQUIRED), ("file", str, _REQUIRED), ("offset", int, _REQUIRED),
             ("length", int, _REQUIRED), ("key", str, _REQUIRED), ("padding", int, 0))

    def __post_init__(self) -> None:
        if min(self.offset, self.length) < 0:
            _fail(CheckpointError, "manifest.ShardRecord",
                  "a shard interval needs a non-negative offset and length",
                  observed={"offset": self.offset, "length": self.length},
                  fix="the manifest entry is damaged")
        validate_shard_filename(self.file)

    @property
    def range(self) -> ShardRange:
        """The interval as a :class:`ShardRange`."""
        return ShardRange(start=self.offset, length=self.length)

    def as_dict(self) -> dict[str, Any]:
        """JSON object of the record."""
        return {name: getattr(self, name) for name, _, _ in self._SPEC}

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> ShardRecord:
        """Inverse of :meth:`as_dict`."""
        return cls(**_decode(payload, cls._SPEC))


@dataclass
class _Coverage:
    """What a set of shard intervals does to a tensor of ``numel`` elements."""

    union: int  # distinct elements covered
    claimed: int  # sum of the lengths (> union when shards overlap)
    past_end: ShardRecord | None  # first shard, by offset, ending beyond the tensor
    overlap: tuple[ShardRecord, ShardRecord] | None  # first pair claiming the same element


def _coverage(shards: list[ShardRecord], numel: int) -> _Coverage:
    """One sweep over the shards in offset order."""
    union = claimed = 0
    reach = 0  # end of the covered prefix of the current run
    holder: ShardRecord | None = None  # shard that reaches furthest so far
    past_end = overlap = None
    for shard in _by_offset(shards):
        end = shard.offset + shard.length
        claimed += shard.length
        if past_end is None and end > numel:
            past_end = shard
        if shard.length == 0:
            continue  # covers nothing and overlaps nothing
        if holder is not None and shard.offset < reach and overlap is None:
            overlap = (holder, shard)  # holder starts no later and reaches past shard.offset
        if end > reach:
            union += end - max(reach, shard.offset)
            reach, holder = end, shard
    return _Coverage(union=union, claimed=claimed, past_end=past_end, overlap=overlap)


@dataclass
class TensorRecord:
    """One global tensor and the shard intervals that make it up
    (``checkpoint/manifest.py:128-281``)."""

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

    _SPEC = (("key", str, _REQUIRED), ("name", str, _REQUIRED), ("global_shape", _int_tuple, _REQUIRED),
             ("dtype", str, _REQUIRED), ("category", str, "model"), ("partition_dim", _optional_int, None),
             ("tensor_parallel_size", int, 1), ("tensor_parallel_rank", int, 0), ("state_name", str, ""))

    @property
    def numel(self) -> int:
        """Elements of the global tensor (1 for a 0-dim shape)."""
        count = 1
        for extent in self.global_shape:
            count *= extent
        return count

    def covered_elements(self) -> int:
        """How many distinct elements the shards cover; overlapping parts count once."""
        return _coverage(self.shards, self.numel).union

    def validate(self) -> None:
        """Refuse shards that reach past the tensor, claim an element twice, or leave
        an element uncovered, checked in that order (``checkpoint/manifest.py:186-229``)."""
        cover = _coverage(self.shards, self.numel)
        if cover.past_end is not None:
            s = cover.past_end
            _fail(CheckpointCorruptionError, "manifest.TensorRecord.validate",
                  f"shard {s.key!r} of {self.key!r} runs past the end of the tensor",
                  expected=f"end <= {self.numel} (shape {tuple(self.global_shape)})",
                  observed=f"[{s.offset}, {s.offset + s.length})",
                  fix="the recorded shape and the shard intervals disagree")
        if cover.claimed != cover.union:
            pair = " and ".join(repr(s.key) for s in cover.overlap or ())
            _fail(CheckpointCorruptionError, "manifest.TensorRecord.validate",
                  f"shards {pair} of {self.key!r} overlap; neither copy of the shared elements "
                  "can be preferred",
                  expected=f"{cover.union} elements claimed once", observed=f"{cover.claimed} claimed",
                  fix="write the checkpoint again with one writer per interval")
        if cover.union != self.numel:
            _fail(IncompleteCheckpointError, "manifest.TensorRecord.validate",
                  f"the shards of {self.key!r} do not cover the whole tensor",
                  expected=f"{self.numel} elements", observed=f"{cover.union} covered",
                  fix="some writer's records are absent; this checkpoint cannot restore the tensor")

    def shards_overlapping(self, wanted: ShardRange) -> list[tuple[ShardRecord, ShardRange]]:
        """``(shard, part of wanted it holds)`` for every shard meeting ``wanted``, in
        offset order: the read plan of one interval (``checkpoint/manifest.py:231-247``)."""
        hits = ((shard, intersect_ranges(shard.range, wanted)) for shard in _by_offset(self.shards))
        return [(shard, part) for shard, part in hits if part is not None]

    def as_dict(self) -> dict[str, Any]:
        """JSON object: the fields, the element count, and the shards in offset order."""
        out: dict[str, Any] = {name: getattr(self, name) for name, _, _ in self._SPEC}
        out["global_shape"] = list(self.global_shape)
        out["numel"] = self.numel
        out["shards"] = [s.as_dict() for s in _by_offset(self.shards)]
        return out

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> TensorRecord:
        """Inverse of :meth:`as_dict` (``numel`` is derived, not read)."""
        shards = [ShardRecord.from_dict(s) for s in payload.get("shards", [])]
        return cls(shards=shards, **_decode(payload, cls._SPEC))


@dataclass(frozen=True)
class FileRecord:
    """Name, SHA-256 and byte size of one payload file (``checkpoint/manifest.py:286-311``)."""

    name: str
    sha256: str
    bytes: int

    _SPEC = (("name", lambda v: validate_shard_filename(str(v)), _REQUIRED), ("sha256", str, _REQUIRED),
             ("bytes", int, _REQUIRED))

    def as_dict(self) -> dict[str, Any]:
        """JSON object of the record."""
        return {f.name: getattr(self, f.name) for f in fields(self)}

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> FileRecord:
        """Inverse of :meth:`as_dict`; the name must follow the payload rule."""
        return cls(**_decode(payload, cls._SPEC))


@dataclass
class CheckpointManifest:
    """Everything a reader needs to find, check and reassemble the saved tensors,
    independent of how many ranks wrote them (``checkpoint/manifest.py:314-561``)."""

    format_version: str = CURRENT_FORMAT_VERSION
    writer_world_size: int = 1
    topology: dict[str, Any] = field(default_factory=dict)
    step: int = 0
    tensors: dict[str, TensorRecord] = field(default_factory=dict)
    files: dict[str, FileRecord] = field(default_factory=dict)
    complete: bool = False
    created_by: str = ""

    _SPEC = (("format_version", str, _REQUIRED), ("created_by", str, ""), ("writer_world_size", int, 1),
             ("topology", dict, {}), ("step", int, 0), ("complete", bool, False))

    def add_shard(self, record: TensorRecord, shard: ShardRecord) -> None:
        """Append ``shard`` to the tensor ``record`` describes, registering the tensor
        (a copy of ``record`` without its shards) the first time it is seen."""
        mine = self.tensors.get(record.key)
        if mine is None:
            mine = TensorRecord(**{f.name: getattr(record, f.name) for f in fields(TensorRecord) if f.name != "shards"})
            self.tensors[record.key] = mine
        elif (mine.global_shape, mine.dtype) != (record.global_shape, record.dtype):
            _fail(CheckpointCorruptionError, "manifest.add_shard",
                  f"writers describe tensor {record.key!r} differently",
                  expected={"shape": tuple(mine.global_shape), "dtype": mine.dtype},
                  observed={"shape": tuple(record.global_shape), "dtype": record.dtype},
                  fix="every writer must save the same model definition")
        mine.shards.append(shard)

    def validate(self) -> None:
        """Refuse a manifest this package cannot trust: an unknown format version, one not
        marked complete, a tensor its shards do not tile exactly, or a shard whose file
        has no integrity record."""
        validate_format_version(self.format_version)
        if not self.complete:
            _fail(IncompleteCheckpointError, "manifest.validate",
                  "manifest is not marked complete: its writer stopped before publishing it",
                  expected=True, observed=self.complete, fix="restore from an earlier checkpoint instead")
        for record in self.tensors.values():
            record.validate()
            unlisted = sorted({s.file for s in record.shards} - set(self.files))
            if unlisted:
                _fail(IncompleteCheckpointError, "manifest.validate",
                      f"{record.key!r} is stored in {unlisted[0]!r}, which has no integrity record",
                      expected=f"one of {sorted(self.files)}", observed=unlisted,
                      fix="the manifest's files table is incomplete")

    def referenced_files(self) -> set[str]:
        """Names of the payload files any tensor is stored in."""
        return {s.file for record in self.tensors.values() for s in record.shards}

    def tensors_by_category(self, category: str) -> dict[str, TensorRecord]:
        """The tensors of one category (``"model"``, ``"optimizer"`` or ``"buffer"``)."""
        return {key: record for key, record in self.tensors.items() if record.category == category}

    def as_dict(self) -> dict[str, Any]:
        """JSON object; tensors and files sorted by key so equal manifests print equal."""
        out: dict[str, Any] = {name: getattr(self, name) for name, _, _ in self._SPEC}
        out["tensors"] = {key: self.tensors[key].as_dict() for key in sorted(self.tensors)}
        out["files"] = {key: self.files[key].as_dict() for key in sorted(self.files)}
        return out

    def to_json(self, *, indent: int | None = 2) -> str:
        """The manifest's text, with keys sorted."""
        return json.dumps(self.as_dict(), indent=indent, sort_keys=True)

    def write(self, path: Path) -> Path:
        """Store :meth:`to_json` at ``path`` (UTF-8) and return the path."""
        target = Path(path)
        target.write_text(self.to_json(), encoding="utf-8")
        return target

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> CheckpointManifest:
        """Inverse of :meth:`as_dict`; any missing or ill-typed field raises
        :class:`CheckpointError`."""
        try:
            tensors = {key: TensorRecord.from_dict(value) for key, value in payload.get("tensors", {}).items()}
            files = {key: FileRecord.from_dict(value) for key, value in payload.get("files", {}).items()}
            return cls(tensors=tensors, files=files, **_decode(payload, cls._SPEC))
        except (KeyError, TypeError, ValueError, AttributeError) as err:
            _fail(CheckpointError, "manifest.from_dict", "manifest is malformed",
                  expected="the fields this format writes", observed=f"{err.__class__.__name__}: {err}",
                  fix="this JSON was not produced as a checkpoint manifest", cause=err)

    @classmethod
    def read(cls, path: Path) -> CheckpointManifest:
        """Parse the manifest at ``path`` (validation is :meth:`validate`'s job)."""
        source = Path(path)
        if not source.is_file():
            _fail(IncompleteCheckpointError, "manifest.read",
                  "no manifest found; it is written last, so the checkpoint never finished",
                  expected=str(source), observed="no such file",
                  fix="pick an earlier checkpoint directory")
        try:
            payload = json.loads(source.read_text(encoding="utf-8"))
        except json.JSONDecodeError as err:
            _fail(CheckpointError, "manifest.read", "manifest is not valid JSON",
                  observed=f"line {err.lineno}, column {err.colno}: {err.msg}",
                  fix="the file is damaged", cause=err)
        if not isinstance(payload, dict):
            _fail(CheckpointError, "manifest.read", "manifest is not a JSON object",
                  observed=type(payload).__name__, fix="the file is damaged")
        return cls.from_dict(payload)
