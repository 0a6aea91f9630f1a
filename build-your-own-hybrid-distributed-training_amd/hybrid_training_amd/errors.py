"""Exception hierarchy and message format shared with the reference.

The class names, their base classes and the message layout produced by
:func:`format_error` follow ``errors.py:45-197`` of the reference, because callers
catch these types and tests match on the text.  :class:`NativeKernelError` is new:
it reports a failure inside ``libhbt.so`` (a HIP launch or runtime error, or a
missing library), which the pure-Python reference cannot produce.
"""

from __future__ import annotations

from typing import Any

__all__ = [
    "CheckpointCorruptionError",
    "CheckpointError",
    "CheckpointTopologyError",
    "CheckpointVersionError",
    "CollectiveError",
    "ConfigurationError",
    "HybridTrainingError",
    "IncompleteCheckpointError",
    "NativeKernelError",
    "ParameterConsistencyError",
    "ShardingError",
    "UnsupportedFeatureError",
    "format_error",
]


def format_error(
    operation: str,
    problem: str,
    *,
    rank: int | None = None,
    world_size: int | None = None,
    expected: Any = None,
    observed: Any = None,
    resolution: str | None = None,
) -> str:
    """Render ``[rank R/W] operation: problem; expected X, observed Y. Fix: hint``.

    Mirrors ``errors.py:45-92``: the rank prefix appears only when a rank is known,
    the expected/observed clause only when either is given, and the fix only when a
    resolution is given.
    """
    parts = []
    if rank is not None:
        parts.append(f"[rank {rank}/{world_size}] " if world_size is not None else f"[rank {rank}] ")
    parts.append(f"{operation}: {problem}")
    if expected is not None or observed is not None:
        parts.append(f"; expected {expected!r}, observed {observed!r}")
    if resolution:
        parts.append(f". Fix: {resolution}")
    return "".join(parts)


class HybridTrainingError(Exception):
    """Root of every error this package raises on purpose."""


class ConfigurationError(HybridTrainingError, ValueError):
    """A configuration object is inconsistent or asks for something unsupported."""


class CollectiveError(HybridTrainingError):
    """A collective was requested in a way that cannot work."""


class ParameterConsistencyError(HybridTrainingError):
    """Parameters that must agree across ranks do not."""


class ShardingError(HybridTrainingError):
    """A flat-parameter, bucket or shard invariant was violated."""


class UnsupportedFeatureError(HybridTrainingError, NotImplementedError):
    """A legal request this library deliberately does not implement."""


class CheckpointError(HybridTrainingError):
    """Base class for checkpoint read/reshard failures."""


class IncompleteCheckpointError(CheckpointError):
    """The shards do not cover the requested elements."""


class CheckpointCorruptionError(CheckpointError):
    """Stored data disagrees with its manifest record."""


class CheckpointVersionError(CheckpointError):
    """A manifest names a format version other than the one this library writes and reads."""


class CheckpointTopologyError(CheckpointError):
    """The saved layout cannot be mapped onto the requested one."""


class NativeKernelError(HybridTrainingError):
    """``libhbt.so`` is missing, mismatched, or one of its kernels failed."""
