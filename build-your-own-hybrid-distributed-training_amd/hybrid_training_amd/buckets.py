"""DDP gradient buckets on one device: layout, pack with the AVG pre-divide, unpack.

Drop-in for the data path of ``parallel/ddp.py``: ``BucketLayout`` and
``GradientBucket`` keep the reference's fields and methods (``ddp.py:111-230``), and
:func:`build_buckets` applies the reference's grouping rule (``ddp.py:397-463``):
walk the parameters in reverse registration order and close a bucket when the next
parameter would push it past ``int(bucket_cap_mb * 2**20)`` bytes, or when dtype or
device changes.

Where the reference copies each gradient into its bucket from a Python hook and
later divides the whole bucket by the group size (``ddp.py:513``,
``distributed/collectives.py:366-367``), :meth:`BucketedGradients.pack` moves every
gradient of every bucket into place and divides it in one launch of the interval
copy kernel: ``bucket[offset + i] = grad[i] / W`` in fp32 true division, which is
bitwise the copy-then-``div_`` of the reference.  :meth:`bind_gradients` then points
each ``param.grad`` at its slice of the bucket (``ddp.py:635-640``), with no copy.
The cross-rank SUM all-reduce of each bucket is not issued: over a trivial group it
is the identity, and over a :meth:`GroupHandle.local_view` group the bucket holds
this rank's pre-divided contribution, ready for it.
"""

from __future__ import annotations

import operator
from collections.abc import Iterable, Iterator, Sequence
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any

import torch
import torch.nn as nn

from . import _native
from .config import DDPConfig
from .errors import ShardingError, UnsupportedFeatureError, format_error
from .groups import GroupHandle

_GRAD = operator.attrgetter("grad")
_DTYPE = operator.attrgetter("dtype")


@dataclass(frozen=True)
class _PackMemo:
    """The launches of the last full pack and the gradients they were built for: every
    gradient's address, dtype and element count, all dense.  Rows depend on nothing
    else, so equal values mean equal rows."""

    ptrs: tuple[int, ...]
    dtypes: tuple[torch.dtype, ...]
    numels: tuple[int, ...]
    divisor: float
    op: int
    plans: tuple[tuple[_native.CopyPlan, torch.dtype, torch.dtype], ...]


def _gradient_signature(params: Sequence[nn.Parameter]) -> tuple | None:
    """``(addresses, dtypes, element counts)`` of the parameters' gradients when every
    one is present and dense, else ``None`` (C-level loops: this runs every step)."""
    grads = list(map(_GRAD, params))
    try:
        ptrs = tuple(map(torch.Tensor.data_ptr, grads))
    except (TypeError, RuntimeError):  # a parameter without a gradient, or a sparse one
        return None
    if not all(map(torch.Tensor.is_contiguous, grads)):
        return None
    return ptrs, tuple(map(_DTYPE, grads)), tuple(map(torch.Tensor.numel, grads))

__all__ = ["BucketLayout", "BucketedGradients", "DDPStatistics", "GradientBucket", "build_buckets"]

_BYTES_PER_MIB = 1024 * 1024


@dataclass(frozen=True)
class BucketLayout:
    """Static description of one bucket (``ddp.py:111-143``)."""

    index: int
    parameter_names: tuple[str, ...]
    offsets: tuple[int, ...]
    numels: tuple[int, ...]
    total_numel: int
    dtype_str: str
    device_str: str

    def as_dict(self) -> dict[str, Any]:
        """JSON form used by cross-rank layout checks."""
        return {
            "index": self.index,
            "parameter_names": list(self.parameter_names),
            "offsets": list(self.offsets),
            "numels": list(self.numels),
            "total_numel": self.total_numel,
            "dtype": self.dtype_str,
        }


class GradientBucket:
    """A flat buffer holding several parameters' gradients (``ddp.py:146-230``)."""

    __slots__ = ("_buffer", "_device", "_dtype", "launched", "layout", "parameters", "pending", "ready", "work")

    def __init__(
        self,
        layout: BucketLayout,
        parameters: Sequence[nn.Parameter],
        dtype: torch.dtype,
        device: torch.device,
    ) -> None:
        self.layout = layout
        self.parameters = tuple(parameters)
        self._dtype = dtype
        self._device = torch.device(device)
        self._buffer: torch.Tensor | None = None
        self.pending: int = len(parameters)
        self.ready: bool = False
        self.launched: bool = False
        self.work: Any = None

    @property
    def buffer(self) -> torch.Tensor:
        """The flat gradient buffer, allocated and zero-filled on first access."""
        if self._buffer is None:
            buffer = torch.empty(self.layout.total_numel, dtype=self._dtype, device=self._device)
            plan = _native.CopyPlan(self._device)
            plan.add_zero(buffer, 0, self.layout.total_numel)
            plan.run(src_dtype=self._dtype, dst_dtype=self._dtype)
            self._buffer = buffer
        return self._buffer

    @property
    def is_allocated(self) -> bool:
        """True once the bucket's storage has been created."""
        return self._buffer is not None

    def view_for(self, position: int) -> torch.Tensor:
        """The bucket slice of the ``position``-th parameter, shaped like it."""
        offset = self.layout.offsets[position]
        numel = self.layout.numels[position]
        return self.buffer[offset : offset + numel].view(self.parameters[position].shape)

    def reset(self) -> None:
        """Prepare for another backward pass."""
        self.pending = len(self.parameters)
        self.ready = False
        self.launched = False
        self.work = None

    def num_bytes(self) -> int:
        """Bytes of the bucket's storage."""
        return self.layout.total_numel * self._dtype.itemsize

    def __repr__(self) -> str:
        return (
            f"GradientBucket(index={self.layout.index}, params={len(self.parameters)}, "
            f"numel={self.layout.total_numel}, pending={self.pending})"
        )


def build_buckets(
    named_parameters: Sequence[tuple[str, nn.Parameter]], bucket_cap_mb: float
) -> list[GradientBucket]:
    """Reverse-order greedy buckets under a byte cap (``ddp.py:397-463``)."""
    cap_bytes = int(bucket_cap_mb * _BYTES_PER_MIB)
    buckets: list[GradientBucket] = []
    current: list[tuple[str, nn.Parameter]] = []
    current_bytes = 0
    current_key: tuple[torch.dtype, torch.device] | None = None

    def close() -> None:
        nonlocal current, current_bytes, current_key
        if not current:
            return
        offsets, numels, cursor = [], [], 0
        for _, param in current:
            offsets.append(cursor)
            numels.append(int(param.numel()))
            cursor += int(param.numel())
        first = current[0][1]
        layout = BucketLayout(
            index=len(buckets),
            parameter_names=tuple(name for name, _ in current),
            offsets=tuple(offsets),
            numels=tuple(numels),
            total_numel=cursor,
            dtype_str=str(first.dtype),
            device_str=str(first.device),
        )
        buckets.append(GradientBucket(layout, [p for _, p in current], first.dtype, first.device))
        current, current_bytes, current_key = [], 0, None

    for name, param in reversed(list(named_parameters)):
        key = (param.dtype, param.device)
        nbytes = int(param.numel()) * param.element_size()
        if current_key is not None and (key != current_key or current_bytes + nbytes > cap_bytes):
            close()
        current_key = key
        current.append((name, param))
        current_bytes += nbytes
    close()
    return buckets


@dataclass
class DDPStatistics:
    """Counters of the bucketing path (``ddp.py:233-263``)."""

    steps: int = 0
    buckets_reduced: int = 0
    bytes_reduced: int = 0
    unused_parameters: tuple[str, ...] = field(default_factory=tuple)

    def as_dict(self) -> dict[str, Any]:
        """JSON form."""
        return {
            "steps": self.steps,
            "buckets_reduced": self.buckets_reduced,
            "bytes_reduced": self.bytes_reduced,
            "unused_parameters": list(self.unused_parameters),
        }


class BucketedGradients:
    """One replica's gradient buckets: pack + AVG pre-divide in one launch, view unpack."""

    def __init__(
        self,
        named_parameters: Sequence[tuple[str, nn.Parameter]],
        group: GroupHandle,
        config: DDPConfig | None = None,
    ) -> None:
        self._config = config or DDPConfig()
        self._group = group
        self._named = [(n, p) for n, p in named_parameters if p.requires_grad]
        if not self._named:
            raise ShardingError(
                format_error(
                    "ddp.DistributedDataParallel",
                    "no trainable parameters were found in the wrapped module; DDP has no gradients to place in buckets",
                    rank=group.global_rank,
                    observed=0,
                    resolution="wrap a module after its parameters exist and require gradients",
                )
            )
        if group.size > 1 and group.process_group is not None:
            raise UnsupportedFeatureError(
                format_error(
                    "ddp.BucketedGradients",
                    "hybrid_training_amd packs one replica's buckets on one device and issues no all-reduce",
                    observed=repr(group),
                )
            )
        for _, p in self._named:
            _native.require_device_tensor(p, "ddp.BucketedGradients")
        self._buckets = build_buckets(self._named, self._config.bucket_cap_mb)
        self._name_of = {id(p): n for n, p in self._named}
        self._all_params = tuple(p for bucket in self._buckets for p in bucket.parameters)
        self._all_bytes = sum(bucket.num_bytes() for bucket in self._buckets)
        self._pack_memo: _PackMemo | None = None
        self._require_backward_grad_sync = True
        self.statistics = DDPStatistics()

    @contextmanager
    def no_sync(self) -> Iterator[None]:
        """Accumulate gradients without packing them (``ddp.py:702-733``).

        Inside, :meth:`pack` and :meth:`synchronize` leave the buckets alone, so the
        micro-batches' gradients keep accumulating in ``param.grad``; the first call
        outside packs (and averages) the accumulated sums.
        """
        previous = self._require_backward_grad_sync
        self._require_backward_grad_sync = False
        try:
            yield
        finally:
            self._require_backward_grad_sync = previous

    @property
    def buckets(self) -> tuple[GradientBucket, ...]:
        """The buckets in launch order."""
        return tuple(self._buckets)

    def bucket_layouts(self) -> list[BucketLayout]:
        """Static layouts in launch order."""
        return [b.layout for b in self._buckets]

    def _divisor(self) -> float:
        # AVG over a trivial group returns before dividing (collectives.py:361-363).
        if self._config.average_gradients and self._group.size > 1:
            return float(self._group.size)
        return 1.0

    def pack(self, buckets: Iterable[int] | None = None) -> None:
        """Copy gradients into their bucket slices, divided by the group size for AVG.

        By default every bucket is packed in one launch.  ``buckets`` selects bucket
        indices instead, so a caller driven by gradient-ready hooks can pack each
        bucket as soon as its last gradient arrives, as the reference copies them
        (``ddp.py:479-523``), and start that bucket's all-reduce while backward runs.
        A parameter without a gradient contributes zeros when
        ``find_unused_parameters`` is set and raises otherwise (``ddp.py:579-615``).
        Inside :meth:`no_sync` it does nothing (``ddp.py:485-489``).
        """
        if not self._require_backward_grad_sync:
            return
        divisor = self._divisor()
        signature = None
        if buckets is None:
            # A full pack over the same dense gradients as the last one reuses its
            # launches: the checks below have nothing new to find, and the per-parameter
            # Python would cost more host time than the kernel takes on a model this size.
            signature = _gradient_signature(self._all_params)
            memo = self._pack_memo
            if (signature is not None and memo is not None and memo.divisor == divisor
                    and signature == (memo.ptrs, memo.dtypes, memo.numels)):
                for plan, src_dtype, dst_dtype in memo.plans:
                    plan.run(src_dtype=src_dtype, dst_dtype=dst_dtype, op=memo.op, divisor=divisor)
                _native.bump_versions([b.buffer for b in self._buckets])
                self.statistics.unused_parameters = ()
                self.statistics.buckets_reduced += len(self._buckets)
                self.statistics.bytes_reduced += self._all_bytes
                return
            selected = self._buckets
        else:
            indices = list(buckets)
            if any(not 0 <= i < len(self._buckets) for i in indices) or len(set(indices)) != len(indices):
                raise ShardingError(
                    format_error("ddp.pack", "bucket indices must be distinct and in range",
                                 expected=f"distinct values in [0, {len(self._buckets)})", observed=indices)
                )
            selected = [self._buckets[i] for i in indices]
        missing: list[str] = []
        # Rows per (device, source dtype, bucket dtype): (source address, destination
        # address, n), source address 0 meaning a zero fill.  Built with plain attribute
        # reads: this loop runs once per step over every parameter.
        rows: dict[tuple[int, torch.dtype, torch.dtype], list[tuple[int, int, int]]] = {}
        # Dense copies of non-contiguous gradients, alive until the plans have run: the
        # rows hold their addresses only.
        dense_copies: list[torch.Tensor] = []
        for bucket in selected:
            buffer = bucket.buffer
            base = buffer.data_ptr()
            item = buffer.element_size()
            bucket_dtype = buffer.dtype
            device_index = buffer.get_device()
            layout = bucket.layout
            for position, param in enumerate(bucket.parameters):
                offset = layout.offsets[position]
                numel = layout.numels[position]
                destination = base + offset * item
                grad = param.grad
                if grad is None:
                    missing.append(self._name_of.get(id(param), f"<param#{position}>"))
                    rows.setdefault((device_index, bucket_dtype, bucket_dtype), []).append((0, destination, numel))
                    continue
                if grad.get_device() != device_index:
                    _native.require_device_tensor(grad, "ddp.pack")
                    raise ShardingError(
                        format_error("ddp.pack", "gradient lives on another device than its bucket",
                                     expected=str(buffer.device), observed=str(grad.device))
                    )
                if not grad.is_contiguous():
                    grad = grad.contiguous()
                    dense_copies.append(grad)
                if grad.numel() != numel:
                    raise ShardingError(
                        format_error("ddp.pack", "gradient size differs from its parameter",
                                     expected=numel, observed=grad.numel())
                    )
                source = grad.data_ptr()
                if source == destination and divisor == 1.0 and grad.dtype == bucket_dtype:
                    continue  # the gradient already is this bucket slice
                rows.setdefault((device_index, grad.dtype, bucket_dtype), []).append((source, destination, numel))
        if missing and not self._config.find_unused_parameters:
            raise ShardingError(
                format_error(
                    "ddp.finish_gradient_synchronization",
                    f"{len(missing)} parameter(s) received no gradient; their buckets would never "
                    "fill, and peers would wait on a reduction that never starts",
                    rank=self._group.global_rank,
                    world_size=self._group.size,
                    observed=missing[:8],
                    resolution=(
                        "pass DDPConfig(find_unused_parameters=True) to reduce zeros for them, "
                        "or set requires_grad=False on parameters the loss does not use"
                    ),
                )
            )
        op = _native.COPY_OP_DIVIDE if divisor != 1.0 else _native.COPY_OP_COPY
        plans = []
        for (device_index, src_dtype, dst_dtype), table in rows.items():
            plan = _native.CopyPlan.from_rows(torch.device("cuda", device_index), table)
            plan.run(src_dtype=src_dtype, dst_dtype=dst_dtype, op=op, divisor=divisor)
            plans.append((plan, src_dtype, dst_dtype))
        # Remembered only for a full pack of gradients that were all present and dense
        # (no temporary copies stand in for them in the rows).
        self._pack_memo = (_PackMemo(*signature, divisor, op, tuple(plans))
                           if signature is not None and not missing and not dense_copies else None)
        if rows:
            _native.bump_versions([b.buffer for b in selected])
        self.statistics.unused_parameters = tuple(missing)
        self.statistics.buckets_reduced += len(selected)
        self.statistics.bytes_reduced += sum(b.num_bytes() for b in selected)

    def bind_gradients(self) -> None:
        """Point every ``param.grad`` at its bucket slice (gradient-as-bucket-view)."""
        for bucket in self._buckets:
            for position, param in enumerate(bucket.parameters):
                param.grad = bucket.view_for(position)
            bucket.reset()

    def synchronize(self) -> None:
        """Pack (with the AVG pre-divide), then rebind gradients to the buckets; inside
        :meth:`no_sync`, nothing (``ddp.py:574-577``)."""
        if not self._require_backward_grad_sync:
            return
        self.pack()
        self.bind_gradients()
        self.statistics.steps += 1
