"""Flat-buffer layout arithmetic and the device copies built on it.

A flat buffer is the concatenation of ``reshape(-1)`` of an ordered list of
tensors, padded with zeros to a multiple of the shard-group size ``G``; shard ``r``
of ``G`` is the half-open element interval ``[r*S, (r+1)*S)`` with
``S = ceil(total / G)``.  Everything in this module except the copy helpers is
integer arithmetic on Python ints.

Names, signatures, error types and messages follow ``utils/tensors.py:58-435`` of
the reference.  The difference is where the bytes move: :func:`flatten_dense_tensors`
and :func:`pad_flat_tensor` run the interval gather-copy kernel of ``libhbt.so``
on the HIP device instead of a Python loop of ``copy_`` calls, and they require
device tensors.
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence
from dataclasses import dataclass

import torch

from . import _native
from .errors import ShardingError, format_error

__all__ = [
    "FlatEntry",
    "ShardRange",
    "build_flat_layout",
    "bytes_of",
    "concat_shard_sizes",
    "even_shard_ranges",
    "flatten_dense_tensors",
    "intersect_ranges",
    "numel_of",
    "pad_flat_tensor",
    "shard_range_for",
    "unflatten_to_views",
]


@dataclass(frozen=True)
class FlatEntry:
    """Placement of one named tensor inside a flat buffer (``utils/tensors.py:58-93``)."""

    name: str
    shape: tuple[int, ...]
    offset: int
    numel: int
    dtype_str: str
    requires_grad: bool = True

    @property
    def end(self) -> int:
        """Index one past the entry's last element."""
        return self.offset + self.numel

    def as_dict(self) -> dict[str, object]:
        """JSON form used by manifests and cross-rank layout checks."""
        return {
            "name": self.name,
            "shape": list(self.shape),
            "offset": self.offset,
            "numel": self.numel,
            "dtype": self.dtype_str,
            "requires_grad": self.requires_grad,
        }


@dataclass(frozen=True)
class ShardRange:
    """Half-open element interval ``[start, start + length)`` (``utils/tensors.py:96-134``)."""

    start: int
    length: int

    def __post_init__(self) -> None:
        if self.start < 0 or self.length < 0:
            raise ShardingError(
                format_error(
                    "tensors.ShardRange",
                    "a range needs a non-negative start and length",
                    observed=(self.start, self.length),
                    resolution="the offset computation that built it went below zero",
                )
            )

    @property
    def end(self) -> int:
        """Index one past the last element."""
        return self.start + self.length

    @property
    def is_empty(self) -> bool:
        """True when the interval holds no element."""
        return self.length == 0

    def as_tuple(self) -> tuple[int, int]:
        """``(start, length)``."""
        return (self.start, self.length)


def build_flat_layout(
    named_tensors: Sequence[tuple[str, torch.Tensor]],
) -> tuple[tuple[FlatEntry, ...], int]:
    """Offsets of ``named_tensors`` concatenated in the given order.

    Offsets are the exclusive prefix sum of the element counts
    (``utils/tensors.py:137-196``); the result is ``(entries, total_numel)``.  An
    empty list or a name given twice raises :class:`ShardingError`.
    """
    if len(named_tensors) == 0:
        raise ShardingError(
            format_error(
                "tensors.build_flat_layout",
                "cannot flatten an empty tensor list",
                expected=">= 1 tensor",
                observed=0,
                resolution="build flat parameters only for modules that own parameters",
            )
        )
    entries: list[FlatEntry] = []
    names: set[str] = set()
    cursor = 0
    for name, tensor in named_tensors:
        if name in names:
            raise ShardingError(
                format_error(
                    "tensors.build_flat_layout",
                    f"duplicate tensor name {name!r}: one tensor (a tied weight?) is listed twice",
                    observed=name,
                    resolution="list every tied tensor once per unit",
                )
            )
        names.add(name)
        count = int(tensor.numel())
        entries.append(
            FlatEntry(
                name=name,
                shape=tuple(int(d) for d in tensor.shape),
                offset=cursor,
                numel=count,
                dtype_str=str(tensor.dtype),
                requires_grad=bool(tensor.requires_grad),
            )
        )
        cursor += count
    return tuple(entries), cursor


def concat_shard_sizes(numel: int, group_size: int) -> tuple[int, int]:
    """``(padded_numel, shard_numel)`` with ``shard_numel = ceil(numel / group_size)``.

    Same contract as ``distributed/collectives.py:894-928``.
    """
    if group_size < 1:
        raise ShardingError(
            format_error(
                "collectives.concat_shard_sizes",
                "group size must be positive",
                expected=">= 1",
                observed=group_size,
                resolution="pass a real group size",
            )
        )
    shard = -(-numel // group_size)
    return shard * group_size, shard


def even_shard_ranges(total_numel: int, num_shards: int) -> tuple[ShardRange, ...]:
    """``num_shards`` equal ranges of ``ceil(total/num_shards)`` elements each.

    The last ranges may run past ``total_numel``; those elements are padding
    (``utils/tensors.py:347-380``).
    """
    if num_shards < 1:
        raise ShardingError(
            format_error(
                "tensors.even_shard_ranges",
                "num_shards must be positive",
                expected=">= 1",
                observed=num_shards,
                resolution="pass the shard-group size",
            )
        )
    length = -(-total_numel // num_shards)
    return tuple(ShardRange(start=index * length, length=length) for index in range(num_shards))


def shard_range_for(total_numel: int, num_shards: int, shard_index: int) -> ShardRange:
    """The padded range of shard ``shard_index`` (``utils/tensors.py:383-407``)."""
    if shard_index < 0 or shard_index >= num_shards:
        raise ShardingError(
            format_error(
                "tensors.shard_range_for",
                "shard index outside the group",
                expected=f"0 <= i < {num_shards}",
                observed=shard_index,
                resolution="use a rank index local to the shard group",
            )
        )
    return even_shard_ranges(total_numel, num_shards)[shard_index]


def intersect_ranges(a: ShardRange, b: ShardRange) -> ShardRange | None:
    """Overlap of two ranges, or ``None`` when they share no element.

    This is the whole of resharding (``utils/tensors.py:410-435``).
    """
    lo = a.start if a.start > b.start else b.start
    hi = a.end if a.end < b.end else b.end
    return ShardRange(start=lo, length=hi - lo) if hi > lo else None


def numel_of(named_tensors: Iterable[tuple[str, torch.Tensor]]) -> int:
    """Total element count of ``(name, tensor)`` pairs."""
    return sum(int(t.numel()) for _, t in named_tensors)


def bytes_of(tensors: Iterable[torch.Tensor]) -> int:
    """Total bytes of ``tensors`` (``numel * element_size``)."""
    return sum(int(t.numel()) * t.element_size() for t in tensors)


def flatten_dense_tensors(
    tensors: Iterable[torch.Tensor], *, out: torch.Tensor | None = None
) -> torch.Tensor:
    """Concatenate ``tensors`` into one 1-D device buffer with one kernel launch.

    Contract of ``utils/tensors.py:199-260``: all tensors share dtype and device,
    ``out`` (when given) has exactly the total element count and is returned.
    """
    items = list(tensors)
    if not items:
        raise ShardingError(
            format_error(
                "tensors.flatten_dense_tensors",
                "nothing to flatten",
                expected=">= 1 tensor",
                observed=0,
                resolution="pass at least one tensor",
            )
        )
    dtype, device = items[0].dtype, items[0].device
    total = 0
    for tensor in items:
        if tensor.dtype != dtype or tensor.device != device:
            raise ShardingError(
                format_error(
                    "tensors.flatten_dense_tensors",
                    "tensors flattened together must share dtype and device",
                    expected=f"{dtype} on {device}",
                    observed=f"{tensor.dtype} on {tensor.device}",
                    resolution="flatten each (dtype, device) group on its own",
                )
            )
        total += int(tensor.numel())
    if out is None:
        out = torch.empty(total, dtype=dtype, device=device)
    elif out.numel() != total:
        raise ShardingError(
            format_error(
                "tensors.flatten_dense_tensors",
                "the output buffer has the wrong size",
                expected=total,
                observed=out.numel(),
                resolution="size it to the sum of the tensors' element counts",
            )
        )
    plan = _native.CopyPlan(out.device)
    cursor = 0
    for tensor in items:
        source = _native.contiguous_source(tensor.detach())
        plan.add(source, 0, out, cursor, int(tensor.numel()))
        cursor += int(tensor.numel())
    plan.run(src_dtype=dtype, dst_dtype=out.dtype)
    return out


def unflatten_to_views(flat: torch.Tensor, entries: Sequence[FlatEntry]) -> list[torch.Tensor]:
    """One view of ``flat`` per entry, shaped like the original tensor.

    Views alias ``flat``: nothing is copied (``utils/tensors.py:263-301``).
    """
    if flat.dim() != 1:
        raise ShardingError(
            format_error(
                "tensors.unflatten_to_views",
                "views are cut from a one-dimensional buffer only",
                observed=flat.dim(),
                resolution="pass buffer.reshape(-1)",
            )
        )
    needed = entries[-1].end if entries else 0
    if flat.numel() < needed:
        raise ShardingError(
            format_error(
                "tensors.unflatten_to_views",
                "the buffer is too short for the layout's last tensor",
                expected=f">= {needed} elements",
                observed=flat.numel(),
                resolution="allocate the padded element count",
            )
        )
    return [flat.narrow(0, e.offset, e.numel).view(e.shape) for e in entries]


def pad_flat_tensor(flat: torch.Tensor, multiple: int, *, value: float = 0.0) -> torch.Tensor:
    """Right-pad a 1-D device tensor with zeros to a multiple of ``multiple``.

    Returns ``flat`` itself when already aligned (``utils/tensors.py:304-344``).  The
    reference only ever pads with zero; that is the only value supported here.
    """
    if flat.dim() != 1:
        raise ShardingError(
            format_error(
                "tensors.pad_flat_tensor",
                "padding applies to one-dimensional tensors only",
                observed=flat.dim(),
                resolution="pad tensor.reshape(-1)",
            )
        )
    if multiple < 1:
        raise ShardingError(
            format_error(
                "tensors.pad_flat_tensor",
                "an alignment multiple must be positive",
                observed=multiple,
                resolution="pass the shard-group size",
            )
        )
    remainder = flat.numel() % multiple
    if remainder == 0:
        return flat
    if value != 0.0:
        raise ShardingError(
            format_error(
                "tensors.pad_flat_tensor",
                "only zero padding is supported, so padding never enters a sum or a norm",
                expected=0.0,
                observed=value,
                resolution="pad with zeros",
            )
        )
    length = int(flat.numel())
    padded = torch.empty(length + multiple - remainder, dtype=flat.dtype, device=flat.device)
    plan = _native.CopyPlan(flat.device)
    plan.add(_native.contiguous_source(flat), 0, padded, 0, length)
    plan.add_zero(padded, length, multiple - remainder)
    plan.run(src_dtype=flat.dtype, dst_dtype=flat.dtype)
    return padded
