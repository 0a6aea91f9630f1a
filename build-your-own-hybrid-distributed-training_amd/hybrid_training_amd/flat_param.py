"""FSDP flat parameter on one device: layout, pack/pad/shard, unpack, gradient share.

Drop-in for the data path of ``FlatParamHandle`` (``parallel/fsdp.py:300-958``) and
the piece helpers around it (``:150-200``, ``:1670-1730``).  Construction, the
properties, the piece layout and the error behaviour are the reference's.  The
tensor work is the interval gather-copy kernel and the local-share kernel of
``libhbt.so``:

* ``_build_shard`` writes this rank's ``S`` elements straight from the parameters
  into the shard, casting to the master dtype and zero-filling padding, in one
  launch; the reference materialises the whole padded buffer first and slices it.
* ``reduce_scatter_gradient`` is the rank's local share of the AVG reduce-scatter:
  cast to the reduce dtype (fp32, bf16, fp16 or fp64), divide by ``G`` and sum over the
  ranks' buffers in rank order with every step rounded to that dtype, widen to the
  fp32 master, zero the padding tail, and in the same pass the squared-norm partials
  of the result, which the next ``clip_grad_norm`` picks up instead of reading the
  shard again (one launch).  Inside ``no_sync`` it accumulates the gradients in the
  reduce dtype instead.  There are no collectives: a group of size 1 is
  the whole job; a :meth:`GroupHandle.local_view` group needs the other ranks'
  buffers resident on this device (``peer_grads``), as the stand-in for the
  reduce-scatter.
* ``full_tensors``/``load_local_pieces``/``local_pieces`` are copy plans over the
  same intervals the reference slices with ``intersect_ranges``.

* ``unshard``/``reshard``/``refill``/``free_full`` manage the gathered buffer's storage
  as the reference does (release the bytes, keep the tensor object and its views,
  refill the same bytes with the version counter kept).  The reference's autograd
  function, whose backward reduce-scatters, is outside this path: the caller hands
  the full gradient to ``reduce_scatter_gradient``.

With ``FSDPConfig.cpu_offload_params`` the shard lives in pinned host memory, as the
reference keeps it on the CPU (``fsdp.py:450-451``): it is built on the device and
copied down, uploaded for every gather and unpack, and ``reduce_scatter_gradient``
returns the gradient shard in pinned host memory (``fsdp.py:763-764``) with its norm
partials still attached, so the clip does not read it back.  The optimizer steps such
a shard on the device by streaming it through (``optim.ShardedOptimizer``).
"""

from __future__ import annotations

import dataclasses
from collections.abc import Sequence
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn as nn

from . import _native
from .config import FSDPConfig, MixedPrecisionConfig, resolve_dtype
from .errors import ShardingError, UnsupportedFeatureError, format_error
from .groups import GroupHandle
from .host_staging import is_host
from .optim import NORM_PARTIALS_ATTR, NormPartials, norm_chunk_elems
from .tensors import FlatEntry, ShardRange, build_flat_layout, intersect_ranges

__all__ = [
    "FlatParamHandle",
    "FlatParameter",
    "PieceLayout",
    "ShardedTensorPiece",
    "optimizer_parameter_layout",
    "reshard_state_dict_pieces",
]

#: Tile sums (doubles, one per 256 shard elements) up to which the local share keeps them
#: in the norm partials' allocation: shards of up to 2 Mi elements.
_SHARED_TILE_SUMS = 8192


@dataclass(frozen=True)
class ShardedTensorPiece:
    """This rank's slice of one parameter in global coordinates (``fsdp.py:150-178``)."""

    name: str
    global_shape: tuple[int, ...]
    offset: int
    data: torch.Tensor

    @property
    def length(self) -> int:
        """Number of owned elements."""
        return int(self.data.numel())

    @property
    def range(self) -> ShardRange:
        """The owned interval of the parameter's row-major flattening."""
        return ShardRange(start=self.offset, length=self.length)


@dataclass(frozen=True)
class PieceLayout:
    """Where a parameter's owned elements sit in this rank's shard (``fsdp.py:181-200``)."""

    name: str
    global_shape: tuple[int, ...]
    parameter_offset: int
    length: int
    local_offset: int


class FlatParameter(nn.Parameter):
    """A rank's flat shard.

    ``gradient_norm_scale_runs`` holds the per-element norm weights as runs
    ``(offset, length, weight)``: the partitioned width over real elements, 0 over
    padding.  ``gradient_norm_scale_vector``, the same weights as one host vector
    (``fsdp.py:456-483``), is built from the runs on first access only.
    """

    @property
    def gradient_norm_scale_vector(self) -> torch.Tensor:
        cached = self.__dict__.get("_norm_scale_vector")
        if cached is None:
            cached = torch.zeros(self.numel(), dtype=torch.float32)
            for offset, length, value in self.__dict__.get("gradient_norm_scale_runs", []):
                cached[offset : offset + length] = value
            self.__dict__["_norm_scale_vector"] = cached
        return cached


def _check_cast(src: torch.dtype, dst: torch.dtype, operation: str) -> None:
    if src != dst and (src, dst) not in _native.COPY_CONVERSIONS:
        raise UnsupportedFeatureError(
            format_error(
                operation,
                "the copy kernel converts only between float64, float32, bfloat16 and float16",
                observed=f"{src} -> {dst}",
            )
        )


class FlatParamHandle:
    """One FSDP unit's flat parameter, sharded over ``shard_group``.

    Args mirror ``parallel/fsdp.py:325-431``.  ``locations`` may be ``None`` when no
    module attributes are to be rebound.  ``keep_originals=True`` leaves the
    original parameters' storage alone (the reference always frees it).
    """

    def __init__(
        self,
        named_parameters: Sequence[tuple[str, nn.Parameter]],
        locations: dict[int, list[tuple[nn.Module, str]]] | None,
        shard_group: GroupHandle,
        config: FSDPConfig,
        mixed_precision: MixedPrecisionConfig,
        device: torch.device,
        *,
        replica_group: GroupHandle | None = None,
        recorder: Any = None,
        keep_originals: bool = False,
    ) -> None:
        if not named_parameters:
            raise ShardingError(
                format_error(
                    "fsdp.FlatParamHandle",
                    "a flat parameter needs at least one parameter to flatten",
                    rank=shard_group.global_rank,
                    observed=0,
                    resolution="skip modules that own no parameters when building units",
                )
            )
        flags = {bool(p.requires_grad) for _, p in named_parameters}
        if len(flags) > 1:
            frozen = [n for n, p in named_parameters if not p.requires_grad]
            raise UnsupportedFeatureError(
                format_error(
                    "fsdp.FlatParamHandle",
                    "mixed requires_grad in one unit: its flat parameter is one tensor with "
                    "one gradient, so it is trained or frozen as a whole",
                    rank=shard_group.global_rank,
                    observed={"frozen": frozen[:8]},
                    resolution="give the frozen parameters a unit of their own",
                )
            )
        if replica_group is not None and replica_group.size > 1:
            raise UnsupportedFeatureError(
                format_error(
                    "fsdp.FlatParamHandle",
                    "hybrid sharding needs a replica all-reduce, and hybrid_training_amd issues no "
                    "collectives",
                    observed=repr(replica_group),
                )
            )
        self._shard_group = shard_group
        self._replica_group = replica_group
        self._config = config
        self._mixed_precision = mixed_precision
        self._device = torch.device(device)
        self._recorder = recorder
        self._requires_grad = next(iter(flags))
        self._names = tuple(name for name, _ in named_parameters)
        self._params = tuple(param for _, param in named_parameters)
        self._locations = (
            {id(p): list(locations.get(id(p), [])) for p in self._params} if locations else {}
        )
        first = self._params[0].dtype
        enabled = mixed_precision.enabled
        self._master_dtype = resolve_dtype(mixed_precision.master_dtype) if enabled else first
        self._compute_dtype = resolve_dtype(mixed_precision.param_dtype) if enabled else first
        self._reduce_dtype = resolve_dtype(mixed_precision.reduce_dtype) if enabled else first

        self._entries, self._total_numel = build_flat_layout(list(named_parameters))
        group = shard_group.size
        self._shard_numel = -(-self._total_numel // group)
        self._padded_numel = self._shard_numel * group
        self._padding = self._padded_numel - self._total_numel

        if config.limit_all_gather_bytes:
            gathered = self._padded_numel * torch.empty(0, dtype=self._compute_dtype).element_size()
            if gathered > config.limit_all_gather_bytes:
                raise ShardingError(
                    format_error(
                        "fsdp.FlatParamHandle",
                        "the gathered buffer of this unit is larger than limit_all_gather_bytes "
                        "allows; while it is gathered, its full copy outweighs what sharding saves",
                        rank=shard_group.global_rank,
                        expected=f"<= {config.limit_all_gather_bytes} bytes",
                        observed=gathered,
                        resolution=(
                            "split the model into smaller units (a lower FSDPConfig.auto_wrap_min_num_params) "
                            "or allow a larger gather (limit_all_gather_bytes)"
                        ),
                    )
                )
        self._offload_params = bool(config.cpu_offload_params)
        self.flat_param = self._build_shard()
        self._attach_gradient_norm_scale()
        self._reduction_count = 0
        self._accumulate_without_reduction = False
        # no_sync accumulation: row q holds rank q's accumulated gradient restricted to
        # this rank's slice, the only part of it this rank's reduce-scatter reads.
        self._grad_accumulator: torch.Tensor | None = None
        self._full: torch.Tensor | None = None
        self._is_sharded = True
        if not keep_originals:
            self._detach_original_parameters()

    # -- construction -----------------------------------------------------------------
    def _build_shard(self) -> nn.Parameter:
        """This rank's shard, packed directly from the parameters (``fsdp.py:434-454``)."""
        shard = torch.empty(self._shard_numel, dtype=self._master_dtype, device=self._device)
        local = self.local_shard_range()
        plans: dict[torch.dtype, _native.CopyPlan] = {}
        for entry, param in zip(self._entries, self._params):
            overlap = intersect_ranges(local, ShardRange(entry.offset, entry.numel))
            if overlap is None:
                continue
            _check_cast(param.dtype, self._master_dtype, "fsdp._build_shard")
            source = _native.contiguous_source(param.detach().to(self._device))
            plan = plans.setdefault(param.dtype, _native.CopyPlan(self._device))
            plan.add(source, overlap.start - entry.offset, shard, overlap.start - local.start,
                     overlap.length)
        padding = intersect_ranges(local, ShardRange(self._total_numel, self._padding))
        zero_plan = plans.setdefault(self._master_dtype, _native.CopyPlan(self._device))
        if padding is not None:
            zero_plan.add_zero(shard, padding.start - local.start, padding.length)
        for dtype, plan in plans.items():
            plan.run(src_dtype=dtype, dst_dtype=self._master_dtype)
        if self._offload_params:
            shard = self._to_host(shard)
        return FlatParameter(shard, requires_grad=self._requires_grad)

    @staticmethod
    def _to_host(tensor: torch.Tensor) -> torch.Tensor:
        """A pinned host copy of a device tensor, complete when this returns."""
        host = torch.empty(tensor.shape, dtype=tensor.dtype, device="cpu", pin_memory=True)
        host.copy_(tensor)
        return host

    def _on_device(self, tensor: torch.Tensor) -> torch.Tensor:
        """``tensor`` itself if it is on the device, else its upload (``fsdp.py:575-577``),
        ordered on the current stream before the launches that read it."""
        tensor = tensor.detach()
        return tensor.to(self._device, non_blocking=True) if is_host(tensor) else tensor

    def _attach_gradient_norm_scale(self) -> None:
        """Per-element norm weights: partitioned width on real elements, 0 on padding.

        Stored as runs (``gradient_norm_scale_runs``), which the norm kernel consumes;
        the reference's host vector (``fsdp.py:456-483``) is built from them only if
        read (:class:`FlatParameter`).
        """
        local = self.local_shard_range()
        runs: list[tuple[int, int, float]] = []

        def append(offset: int, length: int, value: float) -> None:
            # Adjacent elements of equal weight form one run: a pure FSDP shard is one
            # run of real elements and at most one run of padding.
            if runs and runs[-1][2] == value and runs[-1][0] + runs[-1][1] == offset:
                runs[-1] = (runs[-1][0], runs[-1][1] + length, value)
            else:
                runs.append((offset, length, value))

        for entry, param in zip(self._entries, self._params):
            partitioned = self._shard_group.size
            if not getattr(param, "is_tensor_parallel_replicated", True):
                partitioned *= int(getattr(param, "tensor_parallel_group_size", 1))
            overlap = intersect_ranges(local, ShardRange(entry.offset, entry.numel))
            if overlap is not None:
                append(overlap.start - local.start, overlap.length, float(partitioned))
        padding = intersect_ranges(local, ShardRange(self._total_numel, self._padding))
        if padding is not None:
            append(padding.start - local.start, padding.length, 0.0)
        self.flat_param.gradient_norm_scale_runs = runs  # type: ignore[attr-defined]
        self.flat_param.gradient_norm_label = (  # type: ignore[attr-defined]
            f"flat_param[{self._names[0]} .. {self._names[-1]}]"
        )

    def _detach_original_parameters(self) -> None:
        """Deregister and free the originals (``fsdp.py:485-504``)."""
        placeholder = torch.empty(0, dtype=self._compute_dtype, device=self._device)
        for param in self._params:
            for module, attribute in self._locations.get(id(param), []):
                if attribute in module._parameters:
                    del module._parameters[attribute]
                setattr(module, attribute, placeholder)
            param.data = torch.empty(0, dtype=param.dtype, device=param.device)

    # -- properties -------------------------------------------------------------------
    @property
    def entries(self) -> tuple[FlatEntry, ...]:
        """One :class:`FlatEntry` per managed parameter, in flat order."""
        return self._entries

    @property
    def managed_parameters(self) -> tuple[nn.Parameter, ...]:
        """The caller's parameter objects, in flat order."""
        return self._params

    @property
    def names(self) -> tuple[str, ...]:
        """Managed parameter names in flat order."""
        return self._names

    @property
    def device(self) -> torch.device:
        """The device this unit's kernels run on (its shard's, unless the shard is offloaded)."""
        return self._device

    @property
    def total_numel(self) -> int:
        """Elements of all managed parameters together (no padding)."""
        return self._total_numel

    @property
    def padded_numel(self) -> int:
        """``shard_numel * group size``: the total rounded up to whole shards."""
        return self._padded_numel

    @property
    def shard_numel(self) -> int:
        """Elements stored per rank."""
        return self._shard_numel

    @property
    def padding(self) -> int:
        """Padding elements at the end of the flat buffer."""
        return self._padding

    @property
    def shard_group(self) -> GroupHandle:
        """The ranks that each hold one shard of the flat parameter."""
        return self._shard_group

    @property
    def replica_group(self) -> GroupHandle | None:
        """The outer replication group (always trivial or ``None`` here)."""
        return self._replica_group

    @property
    def reduction_count(self) -> int:
        """Gradient reductions performed so far."""
        return self._reduction_count

    @property
    def is_sharded(self) -> bool:
        """Whether only the shard is resident (no gathered full buffer holds storage)."""
        return self._is_sharded

    def local_shard_range(self) -> ShardRange:
        """This rank's interval of the padded flat buffer."""
        return ShardRange(start=self._shard_group.local_rank * self._shard_numel, length=self._shard_numel)

    # -- gather / unpack -------------------------------------------------------------
    def _all_shards(self, peer_shards: Sequence[torch.Tensor] | None, operation: str) -> list[torch.Tensor]:
        if peer_shards is None:
            if self._shard_group.size != 1:
                raise UnsupportedFeatureError(
                    format_error(
                        operation,
                        "materialising the full flat parameter needs every rank's shard; "
                        "hybrid_training_amd issues no all-gather",
                        expected="peer_shards holding all group members' shards",
                        observed=None,
                        resolution="pass peer_shards=[shard_0, ..., shard_G-1] resident on this device",
                    )
                )
            return [self.flat_param.detach()]
        if len(peer_shards) != self._shard_group.size or any(
            s.numel() != self._shard_numel for s in peer_shards
        ):
            raise ShardingError(
                format_error(
                    operation,
                    "peer shards must be one equal-sized shard per group member",
                    expected=f"{self._shard_group.size} x {self._shard_numel}",
                    observed=[int(s.numel()) for s in peer_shards],
                )
            )
        return list(peer_shards)

    def gather_full(self, peer_shards: Sequence[torch.Tensor] | None = None) -> torch.Tensor:
        """The padded full buffer in compute dtype (``fsdp.py:564-591``), built on this device
        from every rank's shard (the all-gather's output)."""
        shards = self._all_shards(peer_shards, "fsdp.gather_full")
        full = torch.empty(self._padded_numel, dtype=self._compute_dtype, device=self._device)
        self._gather_into(full, shards, "fsdp.gather_full")
        self._full = full
        self._is_sharded = False
        return full

    def _gather_into(self, full: torch.Tensor, shards: Sequence[torch.Tensor], operation: str) -> None:
        src_dtype = shards[0].dtype
        _check_cast(src_dtype, self._compute_dtype, operation)
        plan = _native.CopyPlan(self._device)
        for rank, shard in enumerate(shards):
            plan.add(_native.contiguous_source(self._on_device(shard)), 0, full, rank * self._shard_numel,
                     self._shard_numel)
        plan.run(src_dtype=src_dtype, dst_dtype=self._compute_dtype)

    def unshard(self, peer_shards: Sequence[torch.Tensor] | None = None) -> torch.Tensor:
        """Gather the full parameters and bind them to the modules (``fsdp.py:624-634``).

        The reference gathers through an autograd function whose backward
        reduce-scatters the gradient; here the buffer is a plain tensor, and the caller
        passes its gradient to :meth:`reduce_scatter_gradient`.
        """
        full = self.gather_full(peer_shards)
        self.bind_views(full)
        return full

    def reshard(self) -> None:
        """Free the memory of the gathered buffer; the tensor object itself survives (``fsdp.py:636-658``).

        Views of it stay valid objects over zero bytes until :meth:`refill`.
        """
        if self._full is None or self._is_sharded:
            return
        self._full.untyped_storage().resize_(0)
        self._is_sharded = True

    def refill(self, full: torch.Tensor, peer_shards: Sequence[torch.Tensor] | None = None) -> None:
        """Restore the bytes of a buffer freed by :meth:`reshard` (``fsdp.py:660-701``).

        The bytes written are the ones the gather produced, so the tensor's autograd
        version counter is kept, as the reference keeps it.  A buffer that still holds
        its storage is left alone.
        """
        required = self._padded_numel * full.element_size()
        if full.untyped_storage().nbytes() == required:
            return
        shards = self._all_shards(peer_shards, "fsdp.refill")
        with torch.no_grad(), torch.autograd._unsafe_preserve_version_counter(full):
            full.untyped_storage().resize_(required)
            self._gather_into(full.detach(), shards, "fsdp.refill")
        if full is self._full:
            self._is_sharded = False

    def free_full(self) -> None:
        """Drop the gathered buffer and unbind the views (``fsdp.py:783-789``)."""
        if self._full is not None:
            self._full.untyped_storage().resize_(0)
        self._full = None
        self._is_sharded = True
        self.unbind_views()

    def unbind_views(self) -> None:
        """Point the module attributes at empty placeholders (``fsdp.py:613-622``)."""
        placeholder = torch.empty(0, dtype=self._compute_dtype, device=self._device)
        for param in self._params:
            for module, attribute in self._locations.get(id(param), []):
                setattr(module, attribute, placeholder)

    def bind_views(self, full: torch.Tensor) -> None:
        """Rebind each managed module attribute to a view into ``full``; no data moves."""
        sizes = [entry.numel for entry in self._entries]
        if self._padding:
            sizes.append(self._padding)
        pieces = torch.split(full, sizes)
        for index, entry in enumerate(self._entries):
            view = pieces[index].view(entry.shape)
            for module, attribute in self._locations.get(id(self._params[index]), []):
                setattr(module, attribute, view)

    def full_tensors(self, peer_shards: Sequence[torch.Tensor] | None = None) -> dict[str, torch.Tensor]:
        """Every managed parameter, reconstructed by copy (``fsdp.py:912-925``)."""
        shards = [self._on_device(s) for s in self._all_shards(peer_shards, "fsdp.full_tensors")]
        dtype = shards[0].dtype
        out = {e.name: torch.empty(e.shape, dtype=dtype, device=self._device) for e in self._entries}
        plan = _native.CopyPlan(self._device)
        for entry in self._entries:
            dest = out[entry.name].view(-1)
            for rank, shard in enumerate(shards):
                piece = intersect_ranges(
                    ShardRange(rank * self._shard_numel, self._shard_numel),
                    ShardRange(entry.offset, entry.numel),
                )
                if piece is not None:
                    plan.add(_native.contiguous_source(shard.detach()), piece.start - rank * self._shard_numel,
                             dest, piece.start - entry.offset, piece.length)
        plan.run(src_dtype=dtype, dst_dtype=dtype)
        return out

    # -- gradient ---------------------------------------------------------------------
    def reduce_scatter_gradient(
        self, grad_full: torch.Tensor, *, peer_grads: Sequence[torch.Tensor] | None = None
    ) -> torch.Tensor | None:
        """This rank's gradient shard in the master dtype (``fsdp.py:704-769``), padding
        forced to 0.0.

        ``grad_full`` is this rank's padded full gradient.  With a group of size 1
        that is all there is; otherwise ``peer_grads`` must hold every rank's padded
        gradient (``grad_full`` among them, in rank order), summed in rank order.
        The gradients are cast to the reduce dtype (float32, bfloat16, float16 or
        float64), and the AVG divide and the sum are rounded to it, as the reference's
        ops in that dtype are (``collectives.py:593-594``); the result is cast to the
        master dtype (float64, float32, bfloat16 or float16) as ``Tensor.to`` casts.  With
        mixed precision off, all three dtypes are the parameters' own (``fsdp.py:379-392``),
        float64 included.  A float64 master over a narrower reduce dtype is reduced into
        float32 (which holds every value of the reduce dtype exactly) and widened.

        Inside ``no_sync`` (:meth:`set_accumulate_without_reduction`) the gradients
        are accumulated in the reduce dtype instead and ``None`` is returned
        (``fsdp.py:738-745``): the first call keeps a copy of each, later calls add to
        it.  The next call outside ``no_sync`` adds its gradients to the accumulated
        ones and reduces the sums (``fsdp.py:747-749``), in one pass that reads each
        accumulated row once (``hbt_grad_local_share_accumulated``; a float64 reduce
        dtype adds first and then reduces).
        """
        floats = (torch.float32, torch.bfloat16, torch.float16, torch.float64)
        if self._reduce_dtype not in floats or self._master_dtype not in floats:
            raise UnsupportedFeatureError(
                format_error(
                    "fsdp.reduce_scatter_gradient",
                    "the local-share kernel reduces in float64, float32, bfloat16 or float16 into a "
                    "master shard of one of those dtypes",
                    observed=f"reduce {self._reduce_dtype}, master {self._master_dtype}",
                )
            )
        grads = [grad_full] if peer_grads is None else list(peer_grads)
        group = self._shard_group.size
        if len(grads) != group:
            raise UnsupportedFeatureError(
                format_error(
                    "fsdp.reduce_scatter_gradient",
                    "the reduce-scatter needs every rank's gradient; hybrid_training_amd issues no "
                    "collectives",
                    expected=f"{group} gradients (peer_grads)",
                    observed=len(grads),
                )
            )
        for g in grads:
            _native.require_device_tensor(g, "fsdp.reduce_scatter_gradient")
            if g.numel() != self._padded_numel or g.dtype not in floats \
                    or g.dtype != grads[0].dtype or not g.is_contiguous():
                raise ShardingError(
                    format_error(
                        "fsdp.reduce_scatter_gradient",
                        "each gradient must be a dense padded full buffer of one float dtype",
                        expected=f"{self._padded_numel} float64/float32/bfloat16/float16 elements",
                        observed=f"{g.numel()} {g.dtype}",
                    )
                )
        if grads[0].dtype == torch.float64 and self._reduce_dtype != torch.float64:
            raise UnsupportedFeatureError(
                format_error("fsdp.reduce_scatter_gradient",
                             "float64 gradients are reduced in float64 (the kernels narrow only after the sum)",
                             observed=f"reduce dtype {self._reduce_dtype}",
                             resolution="set reduce_dtype to float64, or compute in a narrower dtype")
            )
        local = self.local_shard_range()
        source_rank = self._shard_group.local_rank
        rows = None  # accumulator rows the reduction adds the last micro-batch to
        if self._accumulate_without_reduction:
            self._accumulate(grads, local.start)
            return None
        if self._grad_accumulator is not None:
            if self._reduce_dtype == torch.float64:
                # Reduce the accumulated sums: row q is rank q's total restricted to this
                # rank's slice, so the local share reads it at rank offset 0.
                self._accumulate(grads, local.start)
                accumulator, self._grad_accumulator = self._grad_accumulator, None
                grads = list(accumulator.unbind(0))
                source_rank = 0
            else:
                # The last micro-batch is added to the rows inside the reduction
                # (hbt_grad_local_share_accumulated): the rows are read once, not
                # rewritten and read again.  The kernel only reads them, so they are
                # dropped once it has been queued: a refused launch keeps them.
                rows = self._grad_accumulator
        valid = max(0, min(self._shard_numel, self._total_numel - local.start))
        divisor = float(group) if (self._config.average_gradients and group > 1) else 1.0
        # A float64 master over a narrower reduce dtype: reduce into float32, widen after.
        widen = self._master_dtype == torch.float64 and self._reduce_dtype != torch.float64
        out_dtype = torch.float32 if widen else self._master_dtype
        out = torch.empty(self._shard_numel, dtype=out_dtype, device=self._device)
        chunk = norm_chunk_elems(out_dtype)  # elements per norm partial
        valid_chunks = -(-valid // chunk)
        pad = self._shard_numel - valid
        n_partials = max(1, valid_chunks + -(-pad // chunk))
        n_tiles = max(1, -(-self._shard_numel // 256))
        if n_tiles <= _SHARED_TILE_SUMS:
            # A small shard's launch is bound by host time: the partials and the kernel's
            # tile sums share one allocation (a large shard's tile sums are freed at once).
            partials = torch.empty(n_partials + n_tiles, dtype=torch.float64, device=self._device)
            tile_sums_ptr = partials.data_ptr() + 8 * n_partials
        else:
            partials = torch.empty(n_partials, dtype=torch.float64, device=self._device)
            tile_sums = torch.empty(n_tiles, dtype=torch.float64, device=self._device)
            tile_sums_ptr = tile_sums.data_ptr()
        lib = _native.library()
        args = (group, source_rank, self._shard_numel, valid, _native.dtype_code(grads[0].dtype),
                _native.dtype_code(self._reduce_dtype), divisor, _native.dtype_code(out_dtype),
                out.data_ptr(), partials.data_ptr(), tile_sums_ptr, _native.stream_of(self._device))
        grad_ptrs = _native.pointer_array([g.data_ptr() for g in grads])
        with _native.device_guard(self._device):
            if rows is None:
                status = lib.hbt_grad_local_share_sqnorm(grad_ptrs, *args)
                what = "fsdp.hbt_grad_local_share_sqnorm"
            else:
                status = lib.hbt_grad_local_share_accumulated(
                    grad_ptrs, _native.pointer_array([rows[q].data_ptr() for q in range(group)]), *args)
                what = "fsdp.hbt_grad_local_share_accumulated"
        _native.check(status, what)
        if rows is not None:
            self._grad_accumulator = None
        # The squared-norm partials of the shard's real and padding segments ride on
        # the gradient, so the next clip_grad_norm does not read it again.
        segments = {}
        if valid:
            segments[(0, valid)] = partials[:valid_chunks]
        if pad:
            segments[(valid, pad)] = partials[valid_chunks:n_partials]
        if widen:
            wide = torch.empty(self._shard_numel, dtype=torch.float64, device=self._device)
            plan = _native.CopyPlan(self._device)
            plan.add(out, 0, wide, 0, self._shard_numel)
            plan.run(src_dtype=torch.float32, dst_dtype=torch.float64)
            out, segments = wide, {}  # the partials were chunked for float32; the norm pass sums anew
        if self._offload_params:
            out = self._to_host(out)  # the partials stay on the device and describe the copy
        # The padding is written as exact zeros, so its partials are +0.0.
        zero = frozenset({(valid, pad)}) if pad and (valid, pad) in segments else frozenset()
        setattr(out, NORM_PARTIALS_ATTR, NormPartials(out.data_ptr(), out._version, segments, out.dtype, zero))
        self._reduction_count += 1
        return out

    def _accumulate(self, grads: Sequence[torch.Tensor], start: int) -> None:
        """Add every rank's gradient, restricted to this rank's slice, into the
        accumulator in the reduce dtype (``fsdp.py:738-749``): the cast gradient itself
        on the first call (``clone``, which keeps -0.0), then one addition per element
        rounded to the reduce dtype (``add_``)."""
        shard = self._shard_numel
        flags = 0
        if self._grad_accumulator is None:
            # Rows start on 64-element boundaries so both kernels take their vector paths.
            stride = -(-shard // 64) * 64
            self._grad_accumulator = torch.empty((len(grads), stride), dtype=self._reduce_dtype,
                                                 device=self._device)[:, :shard]
            flags = _native.ACCUMULATE_ASSIGN
        accumulator = self._grad_accumulator
        lib = _native.library()
        step = _native.MAX_TENSORS_PER_LAUNCH
        offset_bytes = start * grads[0].element_size()
        with _native.device_guard(self._device):
            for first in range(0, len(grads), step):
                rows = range(first, min(first + step, len(grads)))
                status = lib.hbt_grad_accumulate(
                    _native.pointer_array([accumulator[q].data_ptr() for q in rows]),
                    _native.pointer_array([grads[q].data_ptr() + offset_bytes for q in rows]),
                    _native.int64_array([shard] * len(rows)),
                    len(rows),
                    _native.dtype_code(self._reduce_dtype),
                    _native.dtype_code(grads[0].dtype),
                    flags,
                    _native.stream_of(self._device),
                )
                _native.check(status, "fsdp.hbt_grad_accumulate")

    def set_accumulate_without_reduction(self, value: bool) -> None:
        """Enable or disable ``no_sync`` accumulation for this unit (``fsdp.py:791-797``).

        While enabled, :meth:`reduce_scatter_gradient` accumulates and returns ``None``;
        the first call after disabling it reduces the accumulated gradients.
        """
        self._accumulate_without_reduction = bool(value)

    @property
    def has_pending_accumulation(self) -> bool:
        """Whether unreduced gradients are held from a ``no_sync`` block (``fsdp.py:799-802``)."""
        return self._grad_accumulator is not None

    def zero_padding_region(self, shard_grad: torch.Tensor) -> None:
        """Zero the padding part of a gradient shard (``fsdp.py:771-781``)."""
        padding = intersect_ranges(self.local_shard_range(), ShardRange(self._total_numel, self._padding))
        if padding is None or padding.length == 0:
            return
        if is_host(shard_grad):  # a host shard's padding takes zeros written from the device
            begin = padding.start - self.local_shard_range().start
            zeros = torch.zeros(padding.length, dtype=shard_grad.dtype, device=self._device)
            shard_grad.detach().view(-1)[begin : begin + padding.length].copy_(zeros)
            return
        plan = _native.CopyPlan(self._device)
        plan.add_zero(shard_grad, padding.start - self.local_shard_range().start, padding.length)
        plan.run(src_dtype=shard_grad.dtype, dst_dtype=shard_grad.dtype)

    # -- state dict -------------------------------------------------------------------
    def local_piece_layout(self) -> list[PieceLayout]:
        """Which elements of which parameters this rank owns (``fsdp.py:810-843``)."""
        local = self.local_shard_range()
        layout: list[PieceLayout] = []
        for entry in self._entries:
            overlap = intersect_ranges(local, ShardRange(entry.offset, entry.numel))
            if overlap is None:
                continue
            layout.append(
                PieceLayout(
                    name=entry.name,
                    global_shape=entry.shape,
                    parameter_offset=overlap.start - entry.offset,
                    length=overlap.length,
                    local_offset=overlap.start - local.start,
                )
            )
        return layout

    def local_pieces(self) -> list[ShardedTensorPiece]:
        """This rank's slice of each owned parameter, copied out (``fsdp.py:845-860``).

        The pieces are on the device, a host-resident shard's too (uploaded first)."""
        shard = self._on_device(self.flat_param)
        layout = self.local_piece_layout()
        datas = [torch.empty(item.length, dtype=shard.dtype, device=shard.device) for item in layout]
        plan = _native.CopyPlan(shard.device)
        for item, data in zip(layout, datas):
            plan.add(shard, item.local_offset, data, 0, item.length)
        plan.run(src_dtype=shard.dtype, dst_dtype=shard.dtype)
        return [
            ShardedTensorPiece(name=item.name, global_shape=item.global_shape,
                               offset=item.parameter_offset, data=data)
            for item, data in zip(layout, datas)
        ]

    def load_local_pieces(self, pieces: dict[str, torch.Tensor]) -> None:
        """Write whole parameter tensors' owned parts into the shard (``fsdp.py:862-910``)."""
        local = self.local_shard_range()
        host = self.flat_param.data if is_host(self.flat_param) else None
        # a host-resident shard is written on the device and copied back
        shard = self._on_device(self.flat_param.data) if host is not None else self.flat_param.data
        plans: dict[torch.dtype, _native.CopyPlan] = {}
        for entry in self._entries:
            tensor = pieces.get(entry.name)
            if tensor is None:
                raise ShardingError(
                    format_error(
                        "fsdp.load_local_pieces",
                        f"no tensor for parameter {entry.name!r} among the pieces to load",
                        rank=self._shard_group.global_rank,
                        observed=sorted(pieces)[:8],
                        resolution="the pieces must come from a model of the same definition",
                    )
                )
            if tuple(tensor.shape) != entry.shape:
                raise ShardingError(
                    format_error(
                        "fsdp.load_local_pieces",
                        f"{entry.name!r} has another shape than the unit's parameter",
                        rank=self._shard_group.global_rank,
                        expected=entry.shape,
                        observed=tuple(tensor.shape),
                        resolution="the pieces must come from a model of the same definition",
                    )
                )
            overlap = intersect_ranges(local, ShardRange(entry.offset, entry.numel))
            if overlap is None:
                continue
            _check_cast(tensor.dtype, shard.dtype, "fsdp.load_local_pieces")
            source = _native.contiguous_source(tensor.detach().to(self._device))
            plans.setdefault(tensor.dtype, _native.CopyPlan(self._device)).add(
                source, overlap.start - entry.offset, shard, overlap.start - local.start, overlap.length
            )
        for dtype, plan in plans.items():
            plan.run(src_dtype=dtype, dst_dtype=shard.dtype)
        if host is not None:
            host.copy_(shard)

    def memory_summary(self) -> dict[str, int]:
        """Per-rank byte counts of this unit (``fsdp.py:927-942``)."""
        element = self.flat_param.element_size()
        grad = self.flat_param.grad
        full = self._full
        return {
            "shard_bytes": self._shard_numel * element,
            "full_bytes": 0 if self._is_sharded or full is None else full.numel() * full.element_size(),
            "grad_shard_bytes": 0 if grad is None else grad.numel() * grad.element_size(),
            "padding_bytes": self._padding * element,
        }

    def metadata(self) -> dict[str, Any]:
        """Deterministic layout description (``fsdp.py:944-952``)."""
        return {
            "names": list(self._names),
            "entries": [entry.as_dict() for entry in self._entries],
            "total_numel": self._total_numel,
            "padded_numel": self._padded_numel,
            "shard_numel": self._shard_numel,
        }

    def __repr__(self) -> str:
        return (
            f"FlatParamHandle(params={len(self._params)}, total_numel={self._total_numel}, "
            f"shard_numel={self._shard_numel}, padding={self._padding}, sharded=True)"
        )


def reshard_state_dict_pieces(
    pieces: Sequence[ShardedTensorPiece], global_shape: tuple[int, ...]
) -> torch.Tensor:
    """Reassemble a parameter from covering pieces placed by offset (``fsdp.py:1670-1730``)."""
    total = 1
    for dim in global_shape:
        total *= dim
    if not pieces:
        raise ShardingError(
            format_error(
                "fsdp.reshard_state_dict_pieces",
                "a tensor cannot be reassembled from zero pieces",
                observed=0,
                resolution="pass every stored piece of the tensor",
            )
        )
    dtype = pieces[0].data.dtype
    device = pieces[0].data.device
    intervals: list[tuple[int, int]] = []
    for piece in pieces:
        end = piece.offset + piece.length
        if end > total:
            raise ShardingError(
                format_error(
                    "fsdp.reshard_state_dict_pieces",
                    f"a piece of {piece.name!r} reaches past the end of the tensor",
                    expected=f"end <= {total}",
                    observed=end,
                    resolution="the pieces and the tensor's shape come from different models",
                )
            )
        intervals.append((piece.offset, end))
    covered, cursor = 0, 0
    for start, end in sorted(intervals):
        if end > cursor:
            covered += end - max(start, cursor)
            cursor = end
    if covered != total:
        missing = total - covered
        raise ShardingError(
            format_error(
                "fsdp.reshard_state_dict_pieces",
                f"{missing} element(s) of {pieces[0].name!r} lie in none of the given pieces",
                expected=f"pieces covering all {total} elements",
                observed=covered,
                resolution="pass every stored piece of the tensor",
            )
        )
    flat = torch.empty(total, dtype=dtype, device=device)
    plan = _native.CopyPlan(device)
    sources = [_native.contiguous_source(piece.data.reshape(-1)) for piece in pieces]
    for index, start, end in _last_writer_segments(intervals):
        plan.add(sources[index], start - pieces[index].offset, flat, start, end - start)
    plan.run(src_dtype=dtype, dst_dtype=dtype)
    return flat.view(global_shape)


def optimizer_parameter_layout(
    units: Sequence[tuple[str, FlatParamHandle]],
) -> list[tuple[nn.Parameter, list[PieceLayout]]]:
    """Each unit's flat shard with the parameter pieces it holds, names carrying the
    unit's prefix (``fsdp.py:1477-1510``).

    Optimizer state has the flat shard's shape, so this layout checkpoints it in the
    parameters' global coordinates and lets it reshard across group sizes.  The
    reference's wrapper walks its module tree for the ``(prefix, handle)`` pairs; the
    caller passes them here, in the order of the optimizer's parameters.
    """
    return [
        (handle.flat_param,
         [dataclasses.replace(item, name=prefix + item.name) for item in handle.local_piece_layout()])
        for prefix, handle in units
    ]


def _last_writer_segments(intervals: Sequence[tuple[int, int]]) -> list[tuple[int, int, int]]:
    """``(index, start, end)`` segments giving every covered element to the last interval
    that covers it.

    Sequential slice assignment in list order lets later pieces overwrite earlier ones
    where they overlap; copying each element once from its last writer gives the same
    result in one launch.  The segments are disjoint and their union is the union of
    the intervals.
    """
    segments: list[tuple[int, int, int]] = []
    claimed: list[tuple[int, int]] = []
    for index in range(len(intervals) - 1, -1, -1):
        start, end = intervals[index]
        cursor = start
        for c_start, c_end in sorted(claimed):
            if c_end <= cursor or c_start >= end:
                continue
            if c_start > cursor:
                segments.append((index, cursor, c_start))
            cursor = max(cursor, c_end)
        if cursor < end:
            segments.append((index, cursor, end))
        claimed.append((start, end))
    return segments
