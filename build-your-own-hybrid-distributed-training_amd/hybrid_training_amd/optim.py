"""Sharded AdamW step and the deterministic global gradient-norm clip on HIP.

Drop-in for ``optim/sharded_optimizer.py`` of the reference.  The public names,
constructor arguments, return types, error classes and the state-dict format are
the reference's; what changes is where the arithmetic runs:

* the weighted fp64 squared norm is one pass of ``hbt_grad_sqnorm_partials``
  (fixed tile-to-block map, fixed reduction trees, so it is bitwise reproducible)
  followed by ``hbt_grad_norm_finalize``, which also derives the clip multiplier
  on the device, so no host round trip sits between the norm and the update;
* the update is ``hbt_adamw_step``, one pass that reads ``p, g, m, v`` once and
  writes ``p, m, v`` once, with torch's per-element arithmetic
  (``torch/optim/adam.py:396-547``) reproduced exactly (see ``include/hbt.h``), on
  fp32 masters or, as torch runs it on bf16 / fp16 tensors, on 2-byte masters.

The inner ``torch.optim.AdamW`` object is still built (``build_inner_optimizer``)
and owns ``param_groups`` and ``state``, so ``state_dict``/``load_state_dict``,
``inner`` and learning-rate changes behave as in the reference; only its
``step`` is never called.

Clip placement.  The clip multiplier never leaves the device: ``clip_grad_norm``
computes the norm and the multiplier there, and no host synchronisation sits between
the norm and the update.  Every multiply is rounded to the gradient's dtype exactly as
the reference's in-place ``grad.mul_`` calls round it, so the parameters and state come
out bitwise the same in all three placements.  What differs is when ``.grad`` changes,
and the HBM traffic of a clipped fp32 step:

* default (the reference's semantics, ``sharded_optimizer.py:333-337``):
  ``clip_grad_norm`` clips ``.grad`` in place before it returns (``hbt_scale_inplace``,
  which reads the multiplier from the device and does nothing when it is 1, as the
  reference multiplies only below 1); the update then reads the clipped gradient.
  4 + 8 + 28 = 40 B/element;
* ``clip_in_step=True``: ``clip_grad_norm`` only records the multiplier; the update
  applies it and writes the clipped gradient back, so ``.grad`` is the reference's after
  ``step()`` but still unclipped between the two calls
  (:meth:`ShardedOptimizer.materialize_pending` clips it at once for a caller that reads
  it in that window; a loss scaler that skips the step does so itself).  36 B/element;
* ``defer_clip=True``: the update applies the multiplier and the gradients are never
  written; ``.grad`` keeps the unclipped values.  32 B/element.
"""

from __future__ import annotations

from collections.abc import Callable, Iterable, Sequence
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch
import torch.nn as nn
from torch.autograd.graph import increment_version

from . import _native
from .config import OptimizerConfig
from .errors import ConfigurationError, ShardingError, UnsupportedFeatureError, format_error
from .groups import GroupHandle
from .host_staging import HostOperand, host_stream, is_host

__all__ = [
    "NormContribution",
    "ShardedOptimizer",
    "build_gradient_norm_contributions",
    "build_inner_optimizer",
    "distributed_gradient_norm",
    "gradient_norm_pass",
]

#: Attribute a deferred loss-scale factor travels under on a gradient tensor.
PENDING_UNSCALE_ATTR = "_hbt_pending_unscale"

#: Attribute under which a kernel that produced a gradient leaves its squared-norm
#: partials (see :class:`NormPartials`).
NORM_PARTIALS_ATTR = "_hbt_norm_partials"


@dataclass
class NormPartials:
    """Unweighted gradient norm partials a producing kernel wrote for its output.

    ``segments`` maps ``(offset, length)`` of the gradient to the partials of that
    segment: one fp64 per norm chunk from the segment's start (32768 elements of an
    fp32 gradient, 65536 of a 2-byte one, 16384 of a float64 one), the layout of
    ``hbt_grad_sqnorm_partials`` with weight 1, each summed in the producer's own fixed
    order.  The record is valid while the gradient keeps the storage address, version
    counter and dtype it had when the partials were written.  Every in-place torch op
    and every kernel of this package that writes the tensor moves the version counter
    and so invalidates it; a write that bypasses the counter (through ``tensor.data``,
    or a foreign kernel writing the storage) does not, and the next norm then uses the
    stale partials.
    """

    data_ptr: int
    version: int
    segments: dict[tuple[int, int], torch.Tensor]
    dtype: torch.dtype = torch.float32
    #: Segments the producer wrote as exact zeros (a flat shard's padding), whose
    #: partials are therefore +0.0: any finite non-negative weight leaves them +0.0.
    zero: frozenset[tuple[int, int]] = frozenset()

    def lookup(self, grad: torch.Tensor, offset: int, length: int) -> torch.Tensor | None:
        """The segment's partials if the record still describes ``grad``."""
        if grad.data_ptr() != self.data_ptr or grad._version != self.version or grad.dtype != self.dtype:
            return None
        return self.segments.get((offset, length))


def _cached_partials(grad: torch.Tensor, offset: int, length: int, unscale: float) -> torch.Tensor | None:
    record = getattr(grad, NORM_PARTIALS_ATTR, None)
    if record is None or unscale != 1.0:
        return None
    return record.lookup(grad, offset, length)


def build_inner_optimizer(
    parameters: Iterable[nn.Parameter], config: OptimizerConfig
) -> torch.optim.Optimizer:
    """The torch optimizer object holding param groups and state (``sharded_optimizer.py:84-126``)."""
    params = [p for p in parameters if p.requires_grad]
    if not params:
        raise ShardingError(
            format_error(
                "optim.build_inner_optimizer",
                "no trainable parameters were supplied to the optimizer",
                observed=0,
                resolution="build the optimizer from the wrapped model's parameters",
            )
        )
    if config.name == "adamw":
        return torch.optim.AdamW(
            params,
            lr=config.learning_rate,
            betas=(float(config.betas[0]), float(config.betas[1])),
            eps=config.eps,
            weight_decay=config.weight_decay,
        )
    return torch.optim.SGD(
        params, lr=config.learning_rate, momentum=config.momentum, weight_decay=config.weight_decay
    )


# ---------------------------------------------------------------------------------------
# gradient norm
# ---------------------------------------------------------------------------------------
def _weight_runs(scale: torch.Tensor) -> list[tuple[int, int, float]]:
    """Run-length form ``(offset, length, weight)`` of a per-element fp64 weight vector."""
    weights = scale.detach().to(device="cpu", dtype=torch.float64).reshape(-1)
    n = int(weights.numel())
    if n == 0:
        return []
    change = torch.nonzero(weights[1:] != weights[:-1]).reshape(-1).tolist()
    starts = [0] + [c + 1 for c in change]
    ends = starts[1:] + [n]
    values = weights[starts].tolist()
    return [(s, e - s, float(w)) for s, e, w in zip(starts, ends, values)]


@dataclass
class NormContribution:
    """One parameter's share of the global squared gradient norm.

    ``scale`` is a scalar weight or a per-element weight vector
    (``sharded_optimizer.py:129-158``).  A vector is piecewise constant over the
    flat layout, so it is kept as runs ``(offset, length, weight)`` and each run
    becomes one weighted segment of the device reduction.  A contribution may be
    built from the runs alone (``scale=None``): an FSDP flat shard is, so a
    billion-element weight vector is never materialised; :meth:`scale_vector`
    builds it on demand.
    """

    parameter: nn.Parameter
    scale: float | torch.Tensor | None
    label: str
    runs: list[tuple[int, int, float]] = field(default_factory=list, repr=False)

    def __post_init__(self) -> None:
        if isinstance(self.scale, torch.Tensor) and not self.runs:
            self.runs = _weight_runs(self.scale)
        if self.scale is None and not self.runs and self.parameter.numel() > 0:
            raise ShardingError(
                format_error(
                    "optim.NormContribution",
                    "a contribution needs a scalar weight, a weight vector or weight runs",
                    observed=self.label,
                )
            )

    @property
    def per_element(self) -> bool:
        """Whether the weights vary per element (a vector or runs)."""
        return not isinstance(self.scale, (int, float))

    def scale_vector(self) -> torch.Tensor:
        """The per-element fp64 weights on the host (built from the runs when needed)."""
        if isinstance(self.scale, torch.Tensor):
            return self.scale
        vector = torch.zeros(self.parameter.numel(), dtype=torch.float64)
        for offset, length, weight in self.runs:
            vector[offset : offset + length] = weight
        return vector

    def segments(self) -> list[tuple[torch.Tensor, int, int, float]]:
        """``(grad, offset, length, weight)`` pieces of this contribution, or ``[]``."""
        grad = self.parameter.grad
        if grad is None:
            return []
        if self.per_element:
            if sum(length for _, length, _ in self.runs) != grad.numel():
                raise ShardingError(
                    format_error(
                        "optim.NormContribution",
                        "the per-element norm weights do not match the gradient length",
                        expected=grad.numel(),
                        observed=sum(length for _, length, _ in self.runs),
                        resolution="rebuild the contributions after re-sharding",
                    )
                )
            return [(grad, offset, length, weight) for offset, length, weight in self.runs]
        return [(grad, 0, int(grad.numel()), float(self.scale))]

    def squared_norm(self, device: torch.device | None = None) -> torch.Tensor:
        """This contribution's weighted squared norm as a 0-dim fp64 device tensor.

        ``device``: where a gradient in host memory is summed (default: its own device,
        or the current HIP device for a host gradient)."""
        grad = self.parameter.grad
        if device is None:
            owner = self.parameter if grad is None else grad
            device = torch.device("cuda", torch.cuda.current_device()) if is_host(owner) else owner.device
        if grad is None:
            return torch.zeros((), dtype=torch.float64, device=device)
        result = gradient_norm_pass(self.segments(), torch.device(device), max_norm=0.0)
        return result.sum


def build_gradient_norm_contributions(
    parameters: Sequence[nn.Parameter], *, world_size: int
) -> list[NormContribution]:
    """Per-parameter norm weights (``sharded_optimizer.py:161-212``).

    A parameter carrying ``gradient_norm_scale_vector`` (an FSDP flat shard) gets
    that vector, in fp64, divided by ``world_size`` (from its run-length form
    ``gradient_norm_scale_runs`` when present); any other parameter gets
    ``partitioned / world_size`` with ``partitioned`` its tensor-parallel width when
    it is not replicated, else 1.
    """
    if world_size < 1:
        raise ShardingError(
            format_error(
                "optim.build_gradient_norm_contributions",
                "world_size must be positive",
                expected=">= 1",
                observed=world_size,
                resolution="the norm is summed over at least one rank",
            )
        )
    contributions: list[NormContribution] = []
    for index, param in enumerate(parameters):
        label = getattr(param, "gradient_norm_label", f"flat_param#{index}")
        # A flat shard built here carries its weights in run-length form, so a
        # billion-element shard's weight vector is neither built nor scanned.
        runs = getattr(param, "gradient_norm_scale_runs", None)
        if runs is not None:
            contributions.append(
                NormContribution(parameter=param, scale=None, label=label,
                                 runs=[(o, n, float(w) / world_size) for o, n, w in runs])
            )
            continue
        vector = getattr(param, "gradient_norm_scale_vector", None)
        if vector is not None:
            contributions.append(
                NormContribution(parameter=param, scale=vector.to(torch.float64) / world_size, label=label)
            )
            continue
        partitioned = 1
        if not getattr(param, "is_tensor_parallel_replicated", True):
            partitioned = int(getattr(param, "tensor_parallel_group_size", 1))
        contributions.append(
            NormContribution(parameter=param, scale=partitioned / world_size, label=f"param#{index}")
        )
    return contributions


class NormResult:
    """Device outputs of one norm pass, in one allocation of four doubles: the weighted
    squared sum, the norm, the double clip multiplier (for float64 gradients), then the
    fp32 clip multiplier (for fp32, bf16 and fp16 gradients) and the int32 non-finite
    flag in the last 8 bytes.  Each field is a 0-dim or 1-element view built on first
    use: a view costs about a microsecond of host time, and a step needs only the
    multiplier's address."""

    __slots__ = ("scalars", "_sum", "_norm", "_grad_mul64", "_grad_mul", "_nonfinite")

    def __init__(self, scalars: torch.Tensor) -> None:
        self.scalars = scalars
        self._sum = self._norm = self._grad_mul64 = self._grad_mul = self._nonfinite = None

    @property
    def sum(self) -> torch.Tensor:
        if self._sum is None:
            self._sum = self.scalars[0]
        return self._sum

    @property
    def norm(self) -> torch.Tensor:
        if self._norm is None:
            self._norm = self.scalars[1]
        return self._norm

    @property
    def grad_mul64(self) -> torch.Tensor:
        if self._grad_mul64 is None:
            self._grad_mul64 = self.scalars[2:3]
        return self._grad_mul64

    @property
    def grad_mul(self) -> torch.Tensor:
        if self._grad_mul is None:
            self._grad_mul = self.scalars[3:].view(torch.float32)[:1]
        return self._grad_mul

    @property
    def nonfinite(self) -> torch.Tensor:
        if self._nonfinite is None:
            self._nonfinite = self.scalars[3:].view(torch.int32)[1:]
        return self._nonfinite

    def multiplier_ptr(self, dtype: torch.dtype) -> int:
        """Device address of the clip multiplier a gradient of ``dtype`` is scaled by: the
        double coefficient for float64 gradients, its fp32 rounding for the others (as
        torch hands a Python-double scalar to kernels of each dtype)."""
        return self.scalars.data_ptr() + (16 if dtype == torch.float64 else 24)


def _mul_ptr(result: NormResult | None, dtype: torch.dtype) -> int | None:
    return None if result is None else result.multiplier_ptr(dtype)


def _pending_unscale(grad: torch.Tensor) -> float:
    return float(getattr(grad, PENDING_UNSCALE_ATTR, 1.0))


def gradient_norm_pass(
    segments: Sequence[tuple[torch.Tensor, int, int, float]],
    device: torch.device,
    *,
    max_norm: float,
    tag: bool = False,
) -> NormResult:
    """Weighted fp64 squared norm of gradient segments, plus the clip multiplier.

    ``segments`` are ``(grad, offset, length, weight)``; a grad tagged with a
    pending loss-scale factor is read through that factor.  Segments are batched
    by (dtype, factor) into launches of at most 16; every launch writes its own
    run of per-chunk partials and one finalize launch sums all of them in a fixed
    order.  With ``tag``, every segment of weight 1 read without a pending factor
    leaves its partials on its gradient (:class:`NormPartials`), so a later pass over
    the unchanged gradient, such as the clip after the loss scaler's overflow check,
    reuses them instead of reading the gradient again.

    A gradient in host memory (a parameter shard kept on the host) is uploaded through
    the device's :class:`~hybrid_training_amd.host_staging.HostStream` and summed there
    chunk by chunk; its partials are the ones the same values would give in HBM at the
    same 16-byte alignment, so the result does not depend on where the gradient lives.
    """
    lib = _native.library()
    batches: dict[tuple[torch.dtype, float], list[tuple[torch.Tensor, int, int, float]]] = {}
    for grad, offset, length, weight in segments:
        if not is_host(grad):
            _native.require_device_tensor(grad, "optim.gradient_norm")
        if grad.dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.float64):
            raise UnsupportedFeatureError(
                format_error(
                    "optim.gradient_norm",
                    "gradients must be float64, float32, bfloat16 or float16",
                    observed=str(grad.dtype),
                )
            )
        if grad.dtype == torch.float64 and _pending_unscale(grad) != 1.0:
            raise UnsupportedFeatureError(
                format_error("optim.gradient_norm",
                             "a float64 gradient is unscaled in place before its norm, not read through "
                             "a deferred factor", resolution="unscale float64 gradients eagerly")
            )
        if not grad.is_contiguous():
            raise ShardingError(
                format_error("optim.gradient_norm", "gradients must be dense", observed=tuple(grad.stride()))
            )
        if length > 0:
            batches.setdefault((grad.dtype, _pending_unscale(grad)), []).append(
                (grad, offset, length, weight)
            )
    launches: list[tuple[torch.dtype, float, list[tuple[torch.Tensor, int, int, float]], int]] = []
    total_partials = 0
    for (dtype, unscale), items in batches.items():
        chunk_elems = norm_chunk_elems(dtype)  # hbt_norm_partials_count's chunk
        for start in range(0, len(items), _native.MAX_TENSORS_PER_LAUNCH):
            chunk = items[start : start + _native.MAX_TENSORS_PER_LAUNCH]
            launches.append((dtype, unscale, chunk, total_partials))
            total_partials += sum(-(-n // chunk_elems) for _, _, n, _ in chunk)
    # sum, norm and the double clip multiplier, then the fp32 multiplier and the flag in
    # the last 8 bytes: one allocation for the finalize's outputs.
    scalars = torch.empty(4, dtype=torch.float64, device=device)
    out = scalars.data_ptr()
    stream = _native.stream_of(device)
    whole = _contiguous_cached_partials(launches, total_partials)
    if whole is not None:
        # Every segment's partials were written by its producer, with weight 1, one after
        # another in one tensor in slot order: the finalize reads them where they are.
        with _native.device_guard(device):
            _native.check(lib.hbt_grad_norm_finalize(whole, total_partials, float(max_norm), out, out + 8,
                                                     out + 24, out + 16, out + 28, stream),
                          "optim.hbt_grad_norm_finalize")
        return NormResult(scalars)
    partials = torch.empty(max(1, total_partials), dtype=torch.float64, device=device)
    fresh: list[tuple[torch.Tensor, int, int, int, int]] = []  # segments whose partials are tagged
    with _native.device_guard(device):
        for dtype, unscale, items, first in launches:
            # Items whose producer already wrote their partials take them from there
            # (times the weight, as the kernel would multiply); the others are summed
            # here, each run of consecutive uncached items in one launch.  Every item
            # keeps its slot, and the finalize sums the slots in a fixed order.
            slot = first
            pending: list[tuple[torch.Tensor, int, int, float]] = []
            pending_first = slot
            for grad, offset, length, weight in items:
                count = int(lib.hbt_norm_partials_count(_native.int64_array([length]), 1, _native.dtype_code(dtype)))
                cached = _cached_partials(grad, offset, length, unscale)
                if tag and cached is None and weight == 1.0 and unscale == 1.0:
                    fresh.append((grad, offset, length, slot, count))
                if cached is not None and cached.numel() == count:
                    _launch_sqnorm(lib, pending, dtype, unscale, partials, pending_first, stream)
                    pending = []
                    target = partials[slot : slot + count]
                    if weight == 1.0:
                        plan = _native.CopyPlan(device)
                        plan.add(cached, 0, target, 0, count)
                        plan.run(src_dtype=torch.float64, dst_dtype=torch.float64)
                    else:
                        torch.mul(cached, weight, out=target)
                    pending_first = slot + count
                elif is_host(grad):
                    _launch_sqnorm(lib, pending, dtype, unscale, partials, pending_first, stream)
                    pending = []
                    _stream_sqnorm(lib, grad, offset, length, weight, dtype, unscale, partials, slot, device)
                    pending_first = slot + count
                else:
                    pending.append((grad, offset, length, weight))
                slot += count
            _launch_sqnorm(lib, pending, dtype, unscale, partials, pending_first, stream)
        status = lib.hbt_grad_norm_finalize(partials.data_ptr(), total_partials, float(max_norm), out, out + 8,
                                            out + 24, out + 16, out + 28, stream)
        _native.check(status, "optim.hbt_grad_norm_finalize")
    records: dict[int, tuple[torch.Tensor, dict[tuple[int, int], torch.Tensor]]] = {}
    for grad, offset, length, slot, count in fresh:
        records.setdefault(id(grad), (grad, {}))[1][(offset, length)] = partials[slot : slot + count]
    for grad, found in records.values():
        record = getattr(grad, NORM_PARTIALS_ATTR, None)
        if record is not None and (record.data_ptr, record.version, record.dtype) == (
                grad.data_ptr(), grad._version, grad.dtype):
            record.segments.update(found)  # keep a producer's still-valid segments
        else:
            setattr(grad, NORM_PARTIALS_ATTR, NormPartials(grad.data_ptr(), grad._version, found, grad.dtype))
    return NormResult(scalars)


def _zero_segment(grad: torch.Tensor, offset: int, length: int) -> bool:
    """Whether ``grad``'s producer wrote the segment as exact zeros (and the record is valid)."""
    record = getattr(grad, NORM_PARTIALS_ATTR, None)
    return record is not None and record.lookup(grad, offset, length) is not None and (offset, length) in record.zero


def _contiguous_cached_partials(launches, total_partials: int) -> int | None:
    """The device address of the partials of every segment in ``launches``, when each
    segment has a producer's partials (:class:`NormPartials`) and no pending unscale,
    has weight 1 or was written as exact zeros (its +0.0 partials times any finite
    non-negative weight are the same +0.0), and those partials lie one after another in
    one tensor in slot order, so a finalize over that address sees what the weighted
    copy into a fresh array would give it."""
    address = None
    expected = None
    for dtype, unscale, items, _ in launches:
        if unscale != 1.0:
            return None
        chunk_elems = norm_chunk_elems(dtype)
        for grad, offset, length, weight in items:
            if weight != 1.0 and not (0.0 <= weight < float("inf") and _zero_segment(grad, offset, length)):
                return None
            cached = _cached_partials(grad, offset, length, unscale)
            if cached is None or cached.numel() != -(-length // chunk_elems) or not cached.is_contiguous():
                return None
            if address is None:
                address = cached.data_ptr()
            elif cached.data_ptr() != expected:
                return None
            expected = cached.data_ptr() + 8 * cached.numel()
    if address is None or expected - address != 8 * total_partials:
        return None
    return address


def norm_chunk_elems(dtype: torch.dtype) -> int:
    """Elements per norm partial: 32768 of an fp32 gradient, 65536 of a 2-byte one,
    16384 of a float64 one."""
    if dtype == torch.float64:
        return 16384
    return 32768 if dtype == torch.float32 else 65536


def _stream_sqnorm(lib, grad, offset, length, weight, dtype, unscale, partials, slot, device) -> None:
    """The partials of a host gradient's segment, from slot ``slot``, summed on ``device``.

    Each staged chunk holds whole norm chunks of the segment and starts at the
    segment's own offset from a 16-byte boundary, so every partial is summed over the
    same elements in the same order as a launch over the segment in HBM would sum it.
    """
    flat = grad.detach().reshape(-1)
    size = flat.element_size()
    lead = ((flat.data_ptr() + offset * size) % 16) // size
    norm_chunk = norm_chunk_elems(dtype)
    staging = host_stream(device)
    chunk = max(norm_chunk, staging.chunk_elems // norm_chunk * norm_chunk)

    def launch(start: int, n: int, staged: list[torch.Tensor], stream: int) -> None:
        _launch_sqnorm(lib, [(staged[0], 0, n, weight)], dtype, unscale, partials, slot + start // norm_chunk, stream)

    staging.run(length, [HostOperand(flat[offset : offset + length])], launch, lead=lead, chunk=chunk)


def _launch_sqnorm(lib, items, dtype, unscale, partials, first, stream) -> None:
    """One ``hbt_grad_sqnorm_partials`` launch writing ``items``' partials from slot ``first``."""
    if not items:
        return
    ptrs = [g.data_ptr() + off * g.element_size() for g, off, _, _ in items]
    status = lib.hbt_grad_sqnorm_partials(
        _native.pointer_array(ptrs),
        _native.int64_array([n for _, _, n, _ in items]),
        _native.double_array([w for _, _, _, w in items]),
        len(items),
        _native.dtype_code(dtype),
        unscale,
        partials.data_ptr() + first * 8,
        stream,
    )
    _native.check(status, "optim.hbt_grad_sqnorm_partials")


def scale_gradients(grads: Sequence[torch.Tensor], dtype: torch.dtype, unscale: float, grad_mul_ptr: int | None,
                    device: torch.device, operation: str) -> None:
    """Multiply dense gradients of one dtype in place by ``unscale`` and ``*grad_mul``,
    each product rounded to the dtype (``hbt_scale_inplace``, or ``hbt_scale_inplace_f64``
    with a double multiplier for float64: the reference's ``grad.mul_``).  Gradients in
    HBM go in launches of up to 16; a gradient in host memory streams through ``device``
    and is final on the host when this returns."""
    lib = _native.library()

    def call(ptrs: list[int], numels: list[int], stream: int) -> None:
        if dtype == torch.float64:
            status = lib.hbt_scale_inplace_f64(_native.pointer_array(ptrs), _native.int64_array(numels), len(ptrs),
                                               float(unscale), grad_mul_ptr, stream)
        else:
            status = lib.hbt_scale_inplace(_native.pointer_array(ptrs), _native.int64_array(numels), len(ptrs),
                                           _native.dtype_code(dtype), unscale, grad_mul_ptr, stream)
        _native.check(status, operation)

    resident = [g for g in grads if not is_host(g)]
    hosted = [g for g in grads if is_host(g)]
    with _native.device_guard(device):
        for start in range(0, len(resident), _native.MAX_TENSORS_PER_LAUNCH):
            chunk = resident[start : start + _native.MAX_TENSORS_PER_LAUNCH]
            call([g.data_ptr() for g in chunk], [g.numel() for g in chunk], _native.stream_of(device))
            increment_version(chunk)
        if hosted:
            staging = host_stream(device)
            for g in hosted:
                staging.run(g.numel(), [HostOperand(g, store=True)],
                            lambda start, n, st, stream: call([st[0].data_ptr()], [n], stream))
            increment_version(hosted)
            staging.synchronize()


def unscale_with_partials(grads: Sequence[torch.Tensor], dtype: torch.dtype, unscale: float, device: torch.device,
                          operation: str) -> None:
    """The loss scaler's in-place unscale, ``g = R(g * unscale)`` rounded to the dtype (the
    reference's ``grad.mul_(inverse)``), fused with the norm partials of the result
    (``hbt_scale_inplace_sqnorm``): each gradient leaves with a :class:`NormPartials`
    record of its whole length, so the overflow check and a following clip read none
    of them again.  A gradient in host memory streams through ``device``, its staged
    chunks placed at its own 16-byte alignment as the norm pass places them, and is
    final on the host when this returns.  Float64 gradients are scaled in double
    (``hbt_scale_inplace_f64``) without partials; the overflow check sums them after."""
    if dtype == torch.float64:
        scale_gradients(grads, dtype, unscale, None, device, operation)
        return
    lib = _native.library()
    code = _native.dtype_code(dtype)
    norm_chunk = norm_chunk_elems(dtype)

    # 2-byte gradients sum 512-element pieces first: the kernel's working storage is
    # PIECES_PER_NORM_CHUNK doubles per partial.
    pieces = _native.PIECES_PER_NORM_CHUNK if dtype in (torch.bfloat16, torch.float16) else 0

    def call(ptrs: list[int], numels: list[int], partials_ptr: int, scratch: torch.Tensor | None,
             stream: int) -> None:
        status = lib.hbt_scale_inplace_sqnorm(_native.pointer_array(ptrs), _native.int64_array(numels), len(ptrs),
                                              code, unscale, partials_ptr,
                                              None if scratch is None else scratch.data_ptr(), stream)
        _native.check(status, operation)

    def count_of(n: int) -> int:
        return -(-n // norm_chunk)

    def piece_scratch(partial_count: int) -> torch.Tensor | None:
        if not pieces or unscale == 1.0:
            return None
        return torch.empty(max(1, partial_count) * pieces, dtype=torch.float64, device=device)

    resident = [g for g in grads if not is_host(g)]
    hosted = [g for g in grads if is_host(g)]
    records: list[tuple[torch.Tensor, torch.Tensor]] = []
    with _native.device_guard(device):
        for start in range(0, len(resident), _native.MAX_TENSORS_PER_LAUNCH):
            chunk = resident[start : start + _native.MAX_TENSORS_PER_LAUNCH]
            counts = [count_of(g.numel()) for g in chunk]
            partials = torch.empty(max(1, sum(counts)), dtype=torch.float64, device=device)
            call([g.data_ptr() for g in chunk], [g.numel() for g in chunk], partials.data_ptr(),
                 piece_scratch(sum(counts)), _native.stream_of(device))
            offset = 0
            for g, k in zip(chunk, counts):
                records.append((g, partials[offset : offset + k]))
                offset += k
        if hosted:
            staging = host_stream(device)
            step = max(norm_chunk, staging.chunk_elems // norm_chunk * norm_chunk)
            for g in hosted:
                flat = g.detach().reshape(-1)
                partials = torch.empty(max(1, count_of(flat.numel())), dtype=torch.float64, device=device)
                lead = (flat.data_ptr() % 16) // flat.element_size()
                # one staged chunk at a time on the staging stream: one scratch of a chunk's size serves all
                scratch = piece_scratch(count_of(min(step, flat.numel())))
                staging.run(
                    flat.numel(), [HostOperand(flat, store=True)],
                    lambda first, n, st, stream, partials=partials, scratch=scratch: call(
                        [st[0].data_ptr()], [n], partials.data_ptr() + 8 * (first // norm_chunk), scratch, stream),
                    lead=lead, chunk=step,
                )
                records.append((g, partials[: count_of(flat.numel())]))
            staging.synchronize()
    increment_version([g for g, _ in records])
    for g, partials in records:
        if g.numel() > 0:
            setattr(g, NORM_PARTIALS_ATTR, NormPartials(g.data_ptr(), g._version, {(0, g.numel()): partials}, g.dtype))


def _check_group(group: GroupHandle, operation: str) -> None:
    if group.size > 1 and group.process_group is not None:
        raise UnsupportedFeatureError(
            format_error(
                operation,
                "hybrid_training_amd computes one rank's share on one device and issues no collectives",
                expected="a trivial group or GroupHandle.local_view(...)",
                observed=repr(group),
                resolution="reduce the fp64 partial sum across ranks outside this library",
            )
        )


def distributed_gradient_norm(
    contributions: Sequence[NormContribution],
    group: GroupHandle,
    *,
    device: torch.device,
    recorder: Any = None,
) -> torch.Tensor:
    """Global L2 norm as a 0-dim fp64 device tensor (``sharded_optimizer.py:215-241``).

    Over a trivial group this is the whole norm.  Over a
    :meth:`GroupHandle.local_view` group it is this rank's share before the
    one-scalar fp64 SUM all-reduce, which this library does not issue.
    """
    _check_group(group, "optim.distributed_gradient_norm")
    segments = [s for c in contributions for s in c.segments()]
    return gradient_norm_pass(segments, torch.device(device), max_norm=0.0).norm


# ---------------------------------------------------------------------------------------
# optimizer
# ---------------------------------------------------------------------------------------
def _grad_signature(params: Sequence[nn.Parameter]) -> tuple[tuple[int, int, int], ...]:
    """Identity, address and version of every gradient: detects any change to them."""
    sig = []
    for p in params:
        g = p.grad
        sig.append((0, 0, 0) if g is None else (id(g), g.data_ptr(), g._version))
    return tuple(sig)


def _write_back_flag(write_back: bool, grad_mul: NormResult | None, unscale: float) -> int:
    """``HBT_STEP_WRITE_GRAD`` when the update must store the scaled gradient: with
    in-place semantics and a multiplier pending.  Without one the gradient is unchanged,
    so neither the store nor, for a host gradient, the copy back is needed."""
    return _native.STEP_WRITE_GRAD if write_back and (grad_mul is not None or unscale != 1.0) else 0


def _adamw_call(lib, pdtype, gdtype, p, g, m, v, numels, unscale, mul_ptr, scalars, flags, stream,
                slot: torch.Tensor | None = None) -> int:
    """One ``hbt_adamw_step`` launch, or ``hbt_adamw_step_f64`` (double scalars) on float64
    parameters; ``p``, ``g``, ``m``, ``v`` are lists of device addresses.  With ``slot`` the
    ``*_slot`` form, whose kernels read the scalars from that device memory."""
    tables = (_native.pointer_array(p), _native.pointer_array(g), _native.pointer_array(m),
              _native.pointer_array(v), _native.int64_array(numels), len(numels))
    if pdtype == torch.float64:
        if slot is not None:
            return lib.hbt_adamw_step_f64_slot(*tables, float(unscale), mul_ptr, *scalars, slot.data_ptr(), flags,
                                               stream)
        return lib.hbt_adamw_step_f64(*tables, float(unscale), mul_ptr, *scalars, flags, stream)
    codes = (_native.dtype_code(pdtype), _native.dtype_code(gdtype))
    if slot is not None:
        return lib.hbt_adamw_step_slot(*tables, *codes, unscale, mul_ptr, *scalars, slot.data_ptr(), flags, stream)
    return lib.hbt_adamw_step(*tables, *codes, unscale, mul_ptr, *scalars, flags, stream)


def _sgd_call(lib, pdtype, gdtype, p, g, buf, numels, unscale, mul_ptr, scalars, flags, stream,
              slot: torch.Tensor | None = None) -> int:
    """One ``hbt_sgd_step`` launch, or ``hbt_sgd_step_f64`` on float64 parameters; with
    ``slot`` the ``*_slot`` form."""
    tables = (_native.pointer_array(p), _native.pointer_array(g),
              None if buf is None else _native.pointer_array(buf), _native.int64_array(numels), len(numels))
    if pdtype == torch.float64:
        if slot is not None:
            return lib.hbt_sgd_step_f64_slot(*tables, float(unscale), mul_ptr, *scalars, slot.data_ptr(), flags,
                                             stream)
        return lib.hbt_sgd_step_f64(*tables, float(unscale), mul_ptr, *scalars, flags, stream)
    codes = (_native.dtype_code(pdtype), _native.dtype_code(gdtype))
    if slot is not None:
        return lib.hbt_sgd_step_slot(*tables, *codes, unscale, mul_ptr, *scalars, slot.data_ptr(), flags, stream)
    return lib.hbt_sgd_step(*tables, *codes, unscale, mul_ptr, *scalars, flags, stream)


def _adamw_scalars(group: dict, step: float) -> tuple[float, ...]:
    """The step's scalars exactly as torch/optim/adam.py:416-547 forms them (Python
    doubles): decay, 1 - beta1, beta2, 1 - beta2, sqrt(bias_correction2), eps, -step_size."""
    lr = float(group["lr"])
    beta1, beta2 = (float(b) for b in group["betas"])
    weight_decay = float(group["weight_decay"])
    bias_correction1 = 1 - beta1**step
    bias_correction2 = 1 - beta2**step
    step_size = lr / bias_correction1
    bias_correction2_sqrt = bias_correction2**0.5
    decay = 1 - lr * weight_decay if weight_decay != 0 else 1.0
    return (decay, 1 - beta1, beta2, 1 - beta2, bias_correction2_sqrt, float(group["eps"]), -step_size)


def _sgd_scalars(group: dict) -> tuple[tuple[float, ...], int]:
    """SGD's scalars (weight_decay, momentum, 1 - dampening, -lr; Python doubles, as torch
    forms them) and the flags they select, without the first-step and write-back flags."""
    lr = float(group["lr"])
    momentum = float(group["momentum"])
    weight_decay = float(group["weight_decay"])
    flags = 0
    if weight_decay != 0:
        flags |= _native.SGD_WEIGHT_DECAY
    if momentum != 0:
        flags |= _native.SGD_MOMENTUM
        if bool(group["nesterov"]):
            flags |= _native.SGD_NESTEROV
    return (weight_decay, momentum, 1 - float(group["dampening"]), -lr), flags


def _next_step(step_t: torch.Tensor) -> float:
    """The value ``step_t += 1`` leaves in an AdamW step counter, formed on the host: a
    torch op on a 0-dim tensor costs a few microseconds, and a step takes one per
    parameter.  For a float32 or float64 counter the exact double sum rounded to its
    dtype is that sum, for every finite count; other dtypes take the torch op."""
    if step_t.dtype == torch.float32:
        return float(np.float32(float(step_t.item()) + 1.0))
    if step_t.dtype == torch.float64:
        return float(step_t.item()) + 1.0
    return float((step_t + 1).item())


def _unrecordable(reason: str) -> UnsupportedFeatureError:
    return UnsupportedFeatureError(
        format_error("optim.ShardedOptimizer.step", f"this step cannot be recorded into a HIP graph: {reason}",
                     resolution="take such steps eagerly; record a step only after an eager one, with the "
                     "gradients, parameters and state in device memory and no pending loss-scale factor")
    )


class _RecordedAdamW:
    """One AdamW launch group recorded into a graph, whose kernels read their scalars
    from ``slot``.  Before each replay, :meth:`prepare` checks that the recorded launch
    still describes the step, formats the new step's scalars, formed as the eager step
    forms them, into the slot's host record (``record``, which the replay copies into the
    slot with every other recorded step's), and returns the action that does what the
    eager step does to the host state: advance the parameters' step counters."""

    def __init__(self, optimizer: "ShardedOptimizer", slot: torch.Tensor, record: int, params: list[nn.Parameter],
                 pdtype: torch.dtype, unscale: float, scalars: tuple[float, ...]) -> None:
        self._optimizer = optimizer
        self._slot = slot
        self._record = record
        self._params = list(params)
        self._grad_ptrs = [p.grad.data_ptr() for p in params]
        self._operands = _RecordedOperands(optimizer, self._params, ("exp_avg", "exp_avg_sq"))
        self._pdtype = pdtype
        self._unscale = unscale
        self._lerp_small = abs(scalars[1]) < 0.5

    @property
    def parameters(self) -> list[nn.Parameter]:
        return self._params

    def prepare(self) -> Callable[[], None]:
        opt = self._optimizer
        groups = _replay_groups(opt, self._params)
        for p, ptr in zip(self._params, self._grad_ptrs):
            _check_recorded_grad(p, ptr)
        states = [opt._optimizer.state[p] for p in self._params]
        self._operands.check(states)
        nexts = [_next_step(s["step"]) for s in states]
        found = {_adamw_scalars(groups[id(p)], step) for p in self._params for step in set(nexts)}
        if len(found) != 1:
            raise _replay_error("the parameters recorded in one launch no longer share their step scalars")
        scalars = found.pop()
        if (abs(scalars[1]) < 0.5) != self._lerp_small:
            raise _replay_error("beta1 crossed 0.5, which selects another recorded kernel")
        lib = _native.library()
        if self._pdtype == torch.float64:
            status = lib.hbt_adamw_scalar_record_f64(self._record, float(self._unscale), *scalars)
        else:
            status = lib.hbt_adamw_scalar_record(self._record, _native.dtype_code(self._pdtype), self._unscale,
                                                 *scalars)
        _native.check(status, "optim.hbt_adamw_scalar_record")

        def commit() -> None:
            for s, value in zip(states, nexts):
                s["step"].fill_(value)  # s["step"] += 1
            self._operands.bump_versions()

        return commit


class _RecordedSgd:
    """One SGD launch group recorded into a graph (see :class:`_RecordedAdamW`); SGD's
    scalars follow the learning rate and the other hyperparameters, not the step."""

    def __init__(self, optimizer: "ShardedOptimizer", slot: torch.Tensor, record: int, params: list[nn.Parameter],
                 pdtype: torch.dtype, unscale: float, flags: int) -> None:
        self._optimizer = optimizer
        self._slot = slot
        self._record = record
        self._params = list(params)
        self._grad_ptrs = [p.grad.data_ptr() for p in params]
        self._operands = _RecordedOperands(optimizer, self._params,
                                           ("momentum_buffer",) if flags & _native.SGD_MOMENTUM else ())
        self._pdtype = pdtype
        self._unscale = unscale
        self._flags = flags

    @property
    def parameters(self) -> list[nn.Parameter]:
        return self._params

    def prepare(self) -> Callable[[], None]:
        opt = self._optimizer
        groups = _replay_groups(opt, self._params)
        for p, ptr in zip(self._params, self._grad_ptrs):
            _check_recorded_grad(p, ptr)
        self._operands.check([opt._optimizer.state[p] for p in self._params])
        found = {_sgd_scalars(groups[id(p)]) for p in self._params}
        if len(found) != 1:
            raise _replay_error("the parameters recorded in one launch no longer share their scalars")
        scalars, flags = found.pop()
        kernel_flags = _native.SGD_WEIGHT_DECAY | _native.SGD_MOMENTUM | _native.SGD_NESTEROV
        if flags != self._flags & kernel_flags:
            raise _replay_error("momentum, Nesterov or weight decay was switched on or off, which selects "
                                "another recorded kernel")
        lib = _native.library()
        if self._pdtype == torch.float64:
            status = lib.hbt_sgd_scalar_record_f64(self._record, float(self._unscale), *scalars, self._flags)
        else:
            status = lib.hbt_sgd_scalar_record(self._record, _native.dtype_code(self._pdtype), self._unscale,
                                               *scalars, self._flags)
        _native.check(status, "optim.hbt_sgd_scalar_record")

        def commit() -> None:
            self._operands.bump_versions()

        return commit


class _RecordedOperands:
    """The parameters and optimizer-state tensors a recorded launch updates, held for the
    graph's life (their memory cannot be handed to another tensor while a replay may
    write it) and checked before each replay: a ``load_state_dict`` places the state in
    new tensors and an assignment to ``.data`` gives a parameter new storage, and a
    replay would still update the recorded ones."""

    def __init__(self, optimizer: "ShardedOptimizer", params: list[nn.Parameter], keys: tuple[str, ...]) -> None:
        self._optimizer = optimizer
        self._params = params
        self._keys = keys
        self._held = self._current()
        self._ptrs = [t.data_ptr() for t in self._held]

    def _current(self) -> list[torch.Tensor]:
        state = self._optimizer._optimizer.state
        return [p.detach() for p in self._params] + [state[p][k] for p in self._params for k in self._keys]

    def bump_versions(self) -> None:
        """Advance the version counters of the tensors a replay updates (a detached
        tensor shares its parameter's counter)."""
        increment_version(self._held)

    def check(self, states: list[dict]) -> None:
        """``states``: the recorded parameters' current state dicts, in order."""
        ptrs = [p.data_ptr() for p in self._params]
        for st in states:
            for key in self._keys:
                tensor = st.get(key)
                if tensor is None:
                    break
                ptrs.append(tensor.data_ptr())
        if ptrs != self._ptrs:
            raise _replay_error("a parameter or its optimizer state is no longer the tensor the step was recorded "
                                "with (a load_state_dict or an assignment to .data since the recording); a replay "
                                "updates the recorded tensors")


def _replay_groups(optimizer: "ShardedOptimizer", params: list[nn.Parameter]) -> dict[int, dict]:
    """The parameter group of each recorded parameter, refusing what the recorded kernels
    cannot do: a parameter no longer in any group, amsgrad or maximize switched on."""
    groups = {id(p): g for g in optimizer._optimizer.param_groups for p in g["params"]}
    for p in params:
        group = groups.get(id(p))
        if group is None:
            raise _replay_error("a recorded parameter is no longer in the optimizer's parameter groups")
        if group.get("amsgrad") or group.get("maximize"):
            raise _replay_error("amsgrad or maximize was switched on; they have no HIP kernel")
    return groups


def _check_recorded_grad(p: nn.Parameter, recorded_ptr: int) -> None:
    if p.grad is None or p.grad.data_ptr() != recorded_ptr:
        raise _replay_error("a parameter's .grad was rebound after recording; a replay reads the gradient "
                            "buffer it was recorded with (write new values into that tensor instead)")
    if _pending_unscale(p.grad) != 1.0:
        raise _replay_error("a loss-scale factor is pending on a recorded gradient (a deferred unscale_); the "
                            "eager step would apply it and the recorded one cannot")


def _replay_error(reason: str) -> UnsupportedFeatureError:
    return UnsupportedFeatureError(
        format_error("graphs.StepGraph.replay", reason, resolution="record the step again")
    )


def _pinned_like(p: torch.Tensor) -> torch.Tensor:
    """An uninitialised host tensor shaped like ``p``, in pinned (page-locked) memory."""
    return torch.empty(p.shape, dtype=p.dtype, device="cpu", pin_memory=True)


#: Where each device state tensor of a large parameter starts, in bytes past the
#: parameter's own address modulo 2 MiB (the alignment of large device allocations).  The
#: fused update streams p, g and the state at the same element index; measured on MI355X
#: with p and g 2 MiB-aligned, AdamW's moments at +4 KiB and +8 KiB ran the update at
#: 6.42-6.54 TB/s against 6.26-6.35 with all four streams at the same offset (and +256 B
#: at 6.11-6.15), so the state is placed there rather than wherever the allocator puts it.
_STATE_SLOTS = {"exp_avg": 0, "exp_avg_sq": 1, "momentum_buffer": 0}
_STATE_OFFSETS = (4096, 8192)
_STATE_PERIOD = 2 << 20
#: Smaller state tensors take a plain allocation (the placement costs up to 2 MiB).
_PLACED_STATE_MIN_BYTES = 64 << 20


def _device_state(p: torch.Tensor, slot: int) -> torch.Tensor:
    """An uninitialised dense device tensor shaped like ``p`` for optimizer state.  A large
    one starts ``_STATE_OFFSETS[slot]`` bytes past ``p``'s address modulo 2 MiB, inside an
    allocation of its own up to 2 MiB longer."""
    nbytes = p.numel() * p.element_size()
    if nbytes < _PLACED_STATE_MIN_BYTES:
        return torch.empty(p.shape, dtype=p.dtype, device=p.device)
    storage = torch.empty(nbytes + _STATE_PERIOD, dtype=torch.uint8, device=p.device)
    shift = (p.data_ptr() + _STATE_OFFSETS[slot] - storage.data_ptr()) % _STATE_PERIOD // 16 * 16
    return storage[shift : shift + nbytes].view(p.dtype).view(p.shape)


class ShardedOptimizer:
    """AdamW or SGD over this rank's shards with a global-norm clip, on HIP kernels.

    Same constructor, methods and properties as ``sharded_optimizer.py:244-499``.
    ``defer_clip`` and ``clip_in_step`` are the additions (see the module docstring);
    with neither, the clip is the reference's in-place clip.  Master parameters
    are float32, bfloat16 or float16, as the reference's flat shards are (the
    parameters' own dtype when mixed precision is off, ``fsdp.py:379-384``); 2-byte
    masters take gradients of their own dtype, fp32 masters fp32 or bf16 gradients.
    With ``config.cpu_offload_state`` the master copies and the optimizer state live in
    pinned host memory, as in the reference, and stream through the device each step
    (:class:`~hybrid_training_amd.host_staging.HostStream`).

    A parameter in host memory (an FSDP shard with ``cpu_offload_params``, which the
    reference steps with torch's optimizer on the CPU) keeps its gradient and its state
    on the host too; its norm pass and its step stream every operand through the device
    and write the results back, bitwise what the same values in HBM give.  The step
    returns once the host copies have landed.  ``amsgrad`` and ``maximize`` have no
    kernel and raise :class:`UnsupportedFeatureError` rather than falling back to torch.
    """

    def __init__(
        self,
        parameters: Iterable[nn.Parameter],
        config: OptimizerConfig,
        *,
        norm_group: GroupHandle,
        device: torch.device,
        recorder: Any = None,
        defer_clip: bool = False,
        clip_in_step: bool = False,
    ) -> None:
        if defer_clip and clip_in_step:
            raise ConfigurationError(
                format_error("optim.ShardedOptimizer",
                             "defer_clip and clip_in_step are two different clip placements; pick one",
                             observed={"defer_clip": defer_clip, "clip_in_step": clip_in_step})
            )
        self._parameters = [p for p in parameters if p.requires_grad]
        self._config = config
        self._norm_group = norm_group
        self._device = torch.device(device)
        self._recorder = recorder
        self._defer_clip = defer_clip
        self._clip_in_step = clip_in_step
        _check_group(norm_group, "optim.ShardedOptimizer")
        for param in self._parameters:
            if not is_host(param):
                _native.require_device_tensor(param, "optim.ShardedOptimizer")
            if param.dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.float64):
                raise UnsupportedFeatureError(
                    format_error(
                        "optim.ShardedOptimizer",
                        "master parameters must be float64, float32, bfloat16 or float16",
                        observed=str(param.dtype),
                    )
                )
        self._offload = bool(config.cpu_offload_state) and self._device.type != "cpu"
        if self._offload:
            # As in the reference, master copies live on the host and the inner
            # optimizer's state is keyed by them; here they and the state sit in
            # pinned memory and stream through the device every step.  A parameter
            # already on the host is its own master.
            self._cpu_parameters = [
                p if is_host(p) else nn.Parameter(_pinned_like(p).copy_(p.detach()), requires_grad=True)
                for p in self._parameters
            ]
            self._optimizer = build_inner_optimizer(self._cpu_parameters, config)
        else:
            self._cpu_parameters = []
            self._optimizer = build_inner_optimizer(self._parameters, config)
        self._host_resident = any(is_host(p) for p in self._parameters)
        self._stream = host_stream(self._device) if (self._offload or self._host_resident) else None
        # host master copy -> the device parameter it follows (state offload only)
        self._device_param = {id(h): d for h, d in zip(self._cpu_parameters, self._parameters) if h is not d}
        self._contributions = build_gradient_norm_contributions(
            self._parameters, world_size=norm_group.size
        )
        self._pending_mul: NormResult | None = None  # the clip multipliers the next step applies
        self._pending_signature: tuple[tuple[int, int, int], ...] | None = None
        # (gradient signature, the norm pass whose non-finite flag describes those gradients)
        self._last_check: tuple[tuple[tuple[int, int, int], ...], NormResult | torch.Tensor] | None = None

    # -- norm and clip ---------------------------------------------------------------
    def _norm(self, max_norm: float) -> tuple[NormResult, tuple[tuple[int, int, int], ...]]:
        """The norm pass over the current gradients, and their signature."""
        segments = [s for c in self._contributions for s in c.segments()]
        result = gradient_norm_pass(segments, self._device, max_norm=max_norm)
        signature = _grad_signature(self._parameters)
        self._last_check = (signature, result)
        return result, signature

    def _scale_grads(self, grad_mul: NormResult | None, unscale_attr: bool) -> None:
        """Apply pending multipliers to the gradients in place (materialisation)."""
        groups: dict[tuple[torch.dtype, float], list[torch.Tensor]] = {}
        for p in self._parameters:
            g = p.grad
            if g is None:
                continue
            _native.require_dense(g, "optim.scale_gradients")
            unscale = _pending_unscale(g) if unscale_attr else 1.0
            groups.setdefault((g.dtype, unscale), []).append(g)
        for (dtype, unscale), grads in groups.items():
            scale_gradients(grads, dtype, unscale, _mul_ptr(grad_mul, dtype), self._device,
                            "optim.hbt_scale_inplace")
        if unscale_attr:
            for p in self._parameters:
                if p.grad is not None and hasattr(p.grad, PENDING_UNSCALE_ATTR):
                    delattr(p.grad, PENDING_UNSCALE_ATTR)

    def materialize_pending(self) -> None:
        """Apply any deferred loss-scale and clip factors to ``.grad`` in place."""
        has_unscale = any(
            p.grad is not None and hasattr(p.grad, PENDING_UNSCALE_ATTR) for p in self._parameters
        )
        mul = self._pending_mul if self._pending_valid() else None
        if has_unscale or mul is not None:
            # Scaling keeps every element's finiteness (a finite norm gives a finite
            # multiplier), so the last norm pass's non-finite flag stays valid.
            flag = self.last_nonfinite_flag()
            self._scale_grads(mul, unscale_attr=has_unscale)
            if flag is not None:
                self._last_check = (_grad_signature(self._parameters), flag)
        self._pending_mul = None
        self._pending_signature = None

    def _pending_valid(self) -> bool:
        if self._pending_mul is None:
            return False
        if self._pending_signature != _grad_signature(self._parameters):
            raise ShardingError(
                format_error(
                    "optim.ShardedOptimizer",
                    "gradients changed between clip_grad_norm() and the step, which applies the "
                    "clip, so the clip can no longer be applied where the reference applies it",
                    resolution="call materialize_pending() right after clip_grad_norm() when the "
                    "gradients are modified before the step: it clips them in place, as the "
                    "reference's clip_grad_norm does",
                )
            )
        return True

    def clip_grad_norm(self, max_norm: float) -> torch.Tensor:
        """Clip to a global L2 norm; return the pre-clip norm (0-dim fp64 device tensor).

        ``max_norm <= 0`` only computes the norm (``sharded_optimizer.py:310-338``).  By
        default ``.grad`` is clipped in place before this returns, as in the reference;
        with ``clip_in_step`` or ``defer_clip`` the next :meth:`step` applies the
        multiplier instead (see the module docstring).
        """
        if self._pending_mul is not None:
            self.materialize_pending()
        result, signature = self._norm(max_norm)
        if max_norm <= 0:
            return result.norm
        self._pending_mul = result
        self._pending_signature = signature
        if not (self._defer_clip or self._clip_in_step):
            self.materialize_pending()  # the reference's grad.mul_(coefficient), on the device
        return result.norm

    def clip_and_step(self, max_norm: float) -> torch.Tensor:
        """``clip_grad_norm(max_norm)`` then ``step()``; returns the pre-clip norm.

        The norm reads the gradients (4 B/element for fp32) and the fused update moves
        28 B/element of p, g, m and v; the default in-place clip adds a read and a write
        of the gradients between them (8 B/element), ``clip_in_step`` a write of the
        clipped gradient by the update (4 B/element), ``defer_clip`` nothing.
        """
        norm = self.clip_grad_norm(max_norm)
        self.step()
        return norm

    @property
    def clips_in_place(self) -> bool:
        """Whether ``.grad`` ends up clipped (and unscaled) as the reference leaves it:
        ``defer_clip=False``.  With ``clip_in_step`` a loss scaler that skips the step
        materialises the pending clip (:meth:`materialize_pending`)."""
        return not self._defer_clip

    def last_nonfinite_flag(self) -> torch.Tensor | None:
        """Device flag from the latest norm pass, if the gradients have not changed since."""
        if self._last_check is None:
            return None
        signature, flag = self._last_check
        if isinstance(flag, NormResult):
            flag = flag.nonfinite
        return flag if signature == _grad_signature(self._parameters) else None

    # -- update ----------------------------------------------------------------------
    def step(self) -> None:
        """One AdamW or SGD step over this rank's shards (``sharded_optimizer.py:340-355``)."""
        mul = self._pending_mul if self._pending_valid() else None
        self._run_step(mul)

    def _run_step(self, grad_mul: NormResult | None) -> None:
        # With in-place semantics the update pass writes the scaled gradient back: the
        # clip, and a loss-scale factor deferred by the scaler, land in .grad as the
        # reference's in-place multiplies would leave them.
        write_back = not self._defer_clip
        if isinstance(self._optimizer, torch.optim.SGD):
            self._run_sgd_step(grad_mul, write_back)
        else:
            self._run_adamw_step(grad_mul, write_back)
        if self._host_resident:
            self._stream.synchronize()  # host parameters, gradients and state are final
        if write_back:
            written = [p.grad for p in self._parameters if p.grad is not None]
            if written and (grad_mul is not None or any(_pending_unscale(g) != 1.0 for g in written)):
                increment_version(written)
            for g in written:
                if hasattr(g, PENDING_UNSCALE_ATTR):
                    delattr(g, PENDING_UNSCALE_ATTR)
        self._pending_mul = None
        self._pending_signature = None

    def _checked_grad(self, p: nn.Parameter, group: dict) -> torch.Tensor | None:
        if group.get("amsgrad") or group.get("maximize"):
            raise UnsupportedFeatureError(
                format_error(
                    "optim.ShardedOptimizer.step",
                    "amsgrad and maximize have no HIP kernel in hybrid_training_amd",
                    observed={"amsgrad": group.get("amsgrad"), "maximize": group.get("maximize")},
                )
            )
        grad = p.grad
        if grad is None:
            return None
        if is_host(p) != is_host(grad):
            raise ShardingError(
                format_error("optim.ShardedOptimizer.step",
                             "a parameter and its gradient must both be in host memory or both on the device",
                             expected=str(p.device), observed=str(grad.device))
            )
        if not is_host(grad):
            _native.require_device_tensor(grad, "optim.ShardedOptimizer.step")
        if grad.shape != p.shape or not grad.is_contiguous() or not p.is_contiguous():
            raise ShardingError(
                format_error(
                    "optim.ShardedOptimizer.step",
                    "gradient and parameter must be dense and of equal shape",
                    expected=tuple(p.shape),
                    observed=tuple(grad.shape),
                )
            )
        if (p.dtype, grad.dtype) not in _native.OPTIMIZER_DTYPES:
            raise UnsupportedFeatureError(
                format_error("optim.ShardedOptimizer.step",
                             "the update kernels take fp32 or bf16 gradients on fp32 masters, and "
                             "gradients of the master's own dtype on bf16 / fp16 masters",
                             observed=f"parameter {p.dtype}, gradient {grad.dtype}")
            )
        return grad

    def _stepped_parameters(self) -> list[tuple[dict, nn.Parameter, torch.Tensor]]:
        """``(group, parameter, gradient)`` of every parameter this step updates.

        Every parameter, its gradient and its existing state are checked here, before
        any state is created or any step counter advances, so a refused step leaves
        the optimizer as it was.
        """
        stepped = []
        for group in self._optimizer.param_groups:
            for p in group["params"]:
                grad = self._checked_grad(self._device_param.get(id(p), p), group)
                if grad is None:
                    continue
                # the state the update reads: AdamW's moments, or SGD's buffer with momentum
                read = (("exp_avg", "exp_avg_sq") if "betas" in group
                        else ("momentum_buffer",) if float(group.get("momentum", 0.0)) != 0.0 else ())
                for key in read:
                    value = self._optimizer.state[p].get(key) if p in self._optimizer.state else None
                    if value is not None:
                        _native.require_dense(value, "optim.ShardedOptimizer.step")
                stepped.append((group, p, grad))
        return stepped

    def _run_adamw_step(self, grad_mul: NormResult | None, write_back: bool) -> None:
        lib = _native.library()
        recording = self._recording_check()
        batches: dict[tuple, list[nn.Parameter]] = {}
        for group, p, grad in self._stepped_parameters():
            state = self._optimizer.state[p]
            if len(state) == 0:
                if recording is not None:
                    raise _unrecordable("the first step creates the optimizer state")
                # Same initial state as torch.optim.Adam._init_group.
                state["step"] = torch.tensor(0.0, dtype=torch.float32)
                state["exp_avg"] = self._zero_state(p, "exp_avg")
                state["exp_avg_sq"] = self._zero_state(p, "exp_avg_sq")
            step_t = state["step"]
            if recording is None:
                step = _next_step(step_t)
                step_t.fill_(step)  # step_t += 1
            else:
                step = _next_step(step_t)  # the step each replay advances to
            key = (_adamw_scalars(group, step), p.dtype, grad.dtype, _pending_unscale(grad))
            batches.setdefault(key, []).append(p)
        stream = _native.stream_of(self._device)
        with _native.device_guard(self._device):
            for (scalars, pdtype, gdtype, unscale), batch in batches.items():
                flags = _write_back_flag(write_back, grad_mul, unscale)
                mul_ptr = _mul_ptr(grad_mul, gdtype)
                for p in batch:
                    if is_host(p):
                        self._streamed_adamw(lib, p, scalars, pdtype, gdtype, unscale, mul_ptr, flags)
                params = [p for p in batch if not is_host(p)]
                slot = None
                if recording is not None and params:
                    slot = recording.new_slot()
                    recording.steps.append(_RecordedAdamW(self, slot, recording.record_address(slot), params,
                                                          pdtype, unscale, scalars))
                for start in range(0, len(params), _native.MAX_TENSORS_PER_LAUNCH):
                    chunk = params[start : start + _native.MAX_TENSORS_PER_LAUNCH]
                    states = [self._optimizer.state[p] for p in chunk]
                    status = _adamw_call(
                        lib, pdtype, gdtype,
                        [p.data_ptr() for p in chunk],
                        [p.grad.data_ptr() for p in chunk],
                        [s["exp_avg"].data_ptr() for s in states],
                        [s["exp_avg_sq"].data_ptr() for s in states],
                        [p.numel() for p in chunk],
                        unscale, mul_ptr, scalars, flags, stream, slot,
                    )
                    _native.check(status, "optim.hbt_adamw_step")
                    increment_version(chunk + [s["exp_avg"] for s in states] + [s["exp_avg_sq"] for s in states])

    def _recording_check(self) -> "_native.GraphRecording | None":
        """The graph recording this step joins, after refusing what a replay cannot repeat."""
        recording = _native.graph_recording()
        if recording is not None and (self._offload or self._host_resident):
            raise _unrecordable("parameters or optimizer state in host memory stream through staging buffers "
                                "and wait for the copies on the host")
        if recording is not None:
            for p in self._parameters:
                if p.grad is not None and _pending_unscale(p.grad) != 1.0:
                    raise _unrecordable("a loss-scaled step decides on the host whether to skip")
        return recording

    def _place_state(self, value: torch.Tensor, reference: torch.Tensor, key: str) -> torch.Tensor:
        """A loaded state tensor on the reference parameter's device and dtype (pinned if host),
        placed as a fresh one would be (:func:`_device_state`)."""
        if is_host(reference):
            return _pinned_like(reference).copy_(value.detach().reshape(reference.shape))
        # The update kernels address numel consecutive elements, so the state is dense.
        placed = _device_state(reference, _STATE_SLOTS.get(key, 0))
        return placed.copy_(value.detach().reshape(reference.shape))

    def _zero_state(self, p: torch.Tensor, key: str) -> torch.Tensor:
        """A zero state tensor beside ``p``: in HBM, or pinned host memory for a host master."""
        if is_host(p):
            return _pinned_like(p).zero_()
        return _device_state(p, _STATE_SLOTS[key]).zero_()

    def _streamed_adamw(self, lib, host_p, scalars, pdtype, gdtype, unscale, mul_ptr, flags) -> None:
        """AdamW on a parameter whose state, or whose every operand, lives on the host.

        With state offload the device parameter and gradient stay in HBM and only
        ``m`` and ``v`` stream, the updated parameter following them to its host copy;
        a host-resident parameter streams ``p``, ``g``, ``m`` and ``v`` and writes back
        ``p``, ``m``, ``v`` and, with in-place semantics, the scaled ``g``.
        """
        dev = self._device_param.get(id(host_p))
        state = self._optimizer.state[host_p]
        m, v = state["exp_avg"], state["exp_avg_sq"]

        def call(p_ptr: int, g_ptr: int, m_ptr: int, v_ptr: int, n: int, stream: int) -> None:
            status = _adamw_call(lib, pdtype, gdtype, [p_ptr], [g_ptr], [m_ptr], [v_ptr], [n], unscale, mul_ptr,
                                 scalars, flags, stream)
            _native.check(status, "optim.hbt_adamw_step")

        if dev is not None:
            grad = dev.grad
            psize, gsize = dev.element_size(), grad.element_size()
            self._stream.run(
                dev.numel(), [HostOperand(m, store=True), HostOperand(v, store=True)],
                lambda start, n, st, stream: call(dev.data_ptr() + psize * start, grad.data_ptr() + gsize * start,
                                                  st[0].data_ptr(), st[1].data_ptr(), n, stream),
                resident=(dev.detach().view(-1), host_p.detach().view(-1)),
            )
            increment_version([dev, host_p, m, v])
            return
        write_grad = bool(flags & _native.STEP_WRITE_GRAD)
        self._stream.run(
            host_p.numel(),
            [HostOperand(host_p, store=True), HostOperand(host_p.grad, store=write_grad),
             HostOperand(m, store=True), HostOperand(v, store=True)],
            lambda start, n, st, stream: call(st[0].data_ptr(), st[1].data_ptr(), st[2].data_ptr(), st[3].data_ptr(),
                                              n, stream),
        )
        increment_version([host_p, m, v])

    def _run_sgd_step(self, grad_mul: NormResult | None, write_back: bool) -> None:
        """torch.optim.SGD's step (``torch/optim/sgd.py``) as one fused kernel per batch."""
        lib = _native.library()
        recording = self._recording_check()
        batches: dict[tuple, list[nn.Parameter]] = {}
        for group, p, grad in self._stepped_parameters():
            # Scalars exactly as torch forms them: Python doubles, rounded to fp32 (and
            # each alpha to a 2-byte parameter dtype inside the kernel's entry point), or
            # kept as doubles for float64 parameters.
            scalars, flags = _sgd_scalars(group)
            if flags & _native.SGD_MOMENTUM:
                state = self._optimizer.state[p]
                if state.get("momentum_buffer") is None:
                    if recording is not None:
                        raise _unrecordable("the first step creates the momentum buffer")
                    # torch starts the buffer as a clone of the first gradient.
                    state["momentum_buffer"] = (_pinned_like(p) if is_host(p)
                                                else _device_state(p, _STATE_SLOTS["momentum_buffer"]))
                    flags |= _native.SGD_FIRST_STEP
            unscale = _pending_unscale(grad)
            key = (scalars, flags | _write_back_flag(write_back, grad_mul, unscale), p.dtype, grad.dtype, unscale)
            batches.setdefault(key, []).append(p)
        stream = _native.stream_of(self._device)
        with _native.device_guard(self._device):
            for (scalars, flags, pdtype, gdtype, unscale), batch in batches.items():
                mul_ptr = _mul_ptr(grad_mul, gdtype)
                for p in batch:
                    if is_host(p):
                        self._streamed_sgd(lib, p, scalars, flags, pdtype, gdtype, unscale, mul_ptr)
                params = [p for p in batch if not is_host(p)]
                slot = None
                if recording is not None and params:
                    slot = recording.new_slot()
                    recording.steps.append(_RecordedSgd(self, slot, recording.record_address(slot), params,
                                                        pdtype, unscale, flags))
                for start in range(0, len(params), _native.MAX_TENSORS_PER_LAUNCH):
                    chunk = params[start : start + _native.MAX_TENSORS_PER_LAUNCH]
                    buffers = ([self._optimizer.state[p]["momentum_buffer"] for p in chunk]
                               if flags & _native.SGD_MOMENTUM else [])
                    status = _sgd_call(lib, pdtype, gdtype, [p.data_ptr() for p in chunk],
                                       [p.grad.data_ptr() for p in chunk],
                                       [b.data_ptr() for b in buffers] if buffers else None,
                                       [p.numel() for p in chunk], unscale, mul_ptr, scalars, flags, stream, slot)
                    _native.check(status, "optim.hbt_sgd_step")
                    increment_version(chunk + buffers)

    def _streamed_sgd(self, lib, host_p, scalars, flags, pdtype, gdtype, unscale, mul_ptr) -> None:
        """SGD on a parameter whose momentum buffer, or whose every operand, lives on the
        host (see :meth:`_streamed_adamw`).  A first step writes the buffer without
        reading it, so the buffer is not uploaded then."""
        dev = self._device_param.get(id(host_p))
        momentum = bool(flags & _native.SGD_MOMENTUM)
        first = bool(flags & _native.SGD_FIRST_STEP)
        buffers = ([HostOperand(self._optimizer.state[host_p]["momentum_buffer"], load=not first, store=True)]
                   if momentum else [])

        def call(p_ptr: int, g_ptr: int, b_ptr: int | None, n: int, stream: int) -> None:
            status = _sgd_call(lib, pdtype, gdtype, [p_ptr], [g_ptr], None if b_ptr is None else [b_ptr], [n],
                               unscale, mul_ptr, scalars, flags, stream)
            _native.check(status, "optim.hbt_sgd_step")

        if dev is not None:
            grad = dev.grad
            psize, gsize = dev.element_size(), grad.element_size()
            self._stream.run(
                dev.numel(), buffers,
                lambda start, n, st, stream: call(dev.data_ptr() + psize * start, grad.data_ptr() + gsize * start,
                                                  st[0].data_ptr() if st else None, n, stream),
                resident=(dev.detach().view(-1), host_p.detach().view(-1)),
            )
            increment_version([dev, host_p, *(b.host for b in buffers)])
            return
        write_grad = bool(flags & _native.STEP_WRITE_GRAD)
        self._stream.run(
            host_p.numel(),
            [HostOperand(host_p, store=True), HostOperand(host_p.grad, store=write_grad), *buffers],
            lambda start, n, st, stream: call(st[0].data_ptr(), st[1].data_ptr(),
                                              st[2].data_ptr() if momentum else None, n, stream),
        )
        increment_version([host_p, *(b.host for b in buffers)])

    def zero_grad(self, *, set_to_none: bool = True) -> None:
        """Release or zero the gradients (``sharded_optimizer.py:357-372``).

        With offloaded state the host master copies never hold gradients (the step
        reads the device gradients), so there is nothing to clear on the host.
        """
        self._pending_mul = None
        self._pending_signature = None
        self._last_check = None
        for param in self._parameters:
            # a deferred unscale factor belongs to the contents being discarded, also
            # when the released tensor object is attached again later
            if param.grad is not None and hasattr(param.grad, PENDING_UNSCALE_ATTR):
                delattr(param.grad, PENDING_UNSCALE_ATTR)
            if set_to_none:
                param.grad = None
            elif param.grad is not None:
                param.grad.detach().zero_()

    # -- introspection -------------------------------------------------------------------
    @property
    def parameters(self) -> tuple[nn.Parameter, ...]:
        """Every parameter a step updates, in construction order."""
        return tuple(self._parameters)

    @property
    def inner(self) -> torch.optim.Optimizer:
        """The torch optimizer object that owns param groups and state."""
        return self._optimizer

    @property
    def norm_group(self) -> GroupHandle:
        """The ranks whose squared-norm partials add up to the global norm."""
        return self._norm_group

    @property
    def contributions(self) -> tuple[NormContribution, ...]:
        """Per-parameter norm weights."""
        return tuple(self._contributions)

    @property
    def learning_rate(self) -> float:
        """Learning rate of the first parameter group."""
        return float(self._optimizer.param_groups[0]["lr"])

    def set_learning_rate(self, value: float) -> None:
        """Set the learning rate of every parameter group."""
        for group in self._optimizer.param_groups:
            group["lr"] = value

    def state_bytes(self) -> int:
        """Bytes of optimizer state held by this rank."""
        total = 0
        for state in self._optimizer.state.values():
            for value in state.values():
                if torch.is_tensor(value):
                    total += value.numel() * value.element_size()
        return total

    # -- serialisation -------------------------------------------------------------------
    def state_dict(self) -> dict[str, Any]:
        """Optimizer state keyed by parameter index (``sharded_optimizer.py:420-443``)."""
        if self._stream is not None:
            self._stream.synchronize()
        inner = self._optimizer.state_dict()
        state: dict[int, dict[str, Any]] = {}
        for index, entry in inner["state"].items():
            state[int(index)] = {
                key: (value.detach().cpu().clone() if torch.is_tensor(value) else value)
                for key, value in entry.items()
            }
        return {
            "param_groups": [
                {k: v for k, v in group.items() if k != "params"} for group in inner["param_groups"]
            ],
            "state": state,
            "num_parameters": len(self._parameters),
        }

    def load_state_dict(self, payload: dict[str, Any]) -> None:
        """Restore :meth:`state_dict` output (``sharded_optimizer.py:445-493``)."""
        expected = len(self._parameters)
        observed = int(payload.get("num_parameters", -1))
        if observed != expected:
            raise ShardingError(
                format_error(
                    "optim.load_state_dict",
                    "the number of parameters with optimizer state in the checkpoint differs "
                    "from this optimizer's, so no state can be assigned",
                    rank=self._norm_group.global_rank,
                    expected=expected,
                    observed=observed,
                    resolution=(
                        "load into a model built and wrapped exactly as the one that saved it"
                    ),
                )
            )
        inner_groups = self._optimizer.state_dict()["param_groups"]
        groups: list[dict[str, Any]] = []
        for saved, existing in zip(payload["param_groups"], inner_groups):
            merged = dict(existing)
            merged.update(saved)
            merged["params"] = existing["params"]
            groups.append(merged)
        target = self._cpu_parameters if self._offload else self._parameters
        state: dict[int, dict[str, Any]] = {}
        for index, entry in payload["state"].items():
            reference = target[int(index)]
            state[int(index)] = {
                key: (
                    self._place_state(value, reference, key)
                    if torch.is_tensor(value) and value.dtype.is_floating_point
                    and value.dim() > 0
                    else value
                )
                for key, value in entry.items()
            }
        self._optimizer.load_state_dict({"state": state, "param_groups": groups})
        self._pending_mul = None
        self._pending_signature = None

    def __repr__(self) -> str:
        return (
            f"ShardedOptimizer({self._config.name}, params={len(self._parameters)}, "
            f"norm_group={self._norm_group.name!r}, offload={self._offload})"
        )

