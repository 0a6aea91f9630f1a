"""Dynamic loss scaler whose gradient passes run on HIP kernels.

Drop-in for ``optim/grad_scaler.py`` of the reference: the state machine
(``unscale_`` / ``step`` / ``update``, growth and backoff, skip on overflow) and the
serialised state are the reference's (``grad_scaler.py:52-298``).  The gradient work
is native:

* ``unscale_`` multiplies each gradient by ``fp32(1/scale)`` in its own dtype, as
  ``grad.mul_(inverse)`` does (by the double ``1/scale`` for float64 gradients, without
  the fused partials below), and in the same pass sums the squares of the result
  into fp64 per-chunk partials (``hbt_scale_inplace_sqnorm``): the finiteness check
  reads those (the sum of squares is non-finite exactly when some element is), and they
  stay on the gradients, so the optimizer's ``clip_grad_norm`` that follows takes the
  norm from them too.  Each gradient is read and written once.
* With ``defer_unscale=True`` the multiply is not applied to ``.grad`` here; the
  factor travels with each gradient tensor and the optimizer's norm pass and fused
  update pass apply it while they read the gradient, rounding the product to the
  gradient's dtype as the in-place multiply would, so the results are bitwise those
  of the in-place sequence and a clipped, loss-scaled step costs one norm pass and one
  update pass.  ``unscale_`` then returns a lazily evaluated flag, and ``step`` takes
  the overflow decision from the optimizer's norm pass when it covered the same
  gradients.  An optimizer with in-place semantics (``defer_clip=False``) writes the
  unscaled, clipped gradients back in its ``clip_grad_norm`` (by default) or its step
  (``clip_in_step``), or, when the step is skipped, here.  Float64 gradients are always
  unscaled at once, in double.  A factor still pending when ``unscale_`` is called again is applied in place
  first (two calls multiply twice, as in the reference), and ``step`` applies pending
  factors in place before handing the gradients to any optimizer other than
  ``ShardedOptimizer``, which would not read them.

The overflow decision is taken over this device's gradients only; the one-element
MAX all-reduce that agrees on it across ranks (``grad_scaler.py:191-199``) is not
issued.
"""

from __future__ import annotations

import logging
from collections.abc import Iterable, Sequence
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn as nn

from . import _native
from .config import GradScalerConfig
from .errors import UnsupportedFeatureError, format_error
from .groups import GroupHandle
from .host_staging import is_host
from .optim import PENDING_UNSCALE_ATTR, ShardedOptimizer, gradient_norm_pass, scale_gradients, unscale_with_partials

__all__ = ["GradScaler", "GradScalerState"]

_LOGGER = logging.getLogger(__name__)


@dataclass
class GradScalerState:
    """Serialisable scaler state (``grad_scaler.py:52-92``)."""

    scale: float
    growth_tracker: int = 0
    total_steps: int = 0
    skipped_steps: int = 0

    def as_dict(self) -> dict[str, float]:
        """JSON form."""
        return {
            "scale": float(self.scale),
            "growth_tracker": int(self.growth_tracker),
            "total_steps": int(self.total_steps),
            "skipped_steps": int(self.skipped_steps),
        }

    @classmethod
    def from_dict(cls, payload: dict[str, Any]) -> GradScalerState:
        """Inverse of :meth:`as_dict`."""
        return cls(
            scale=float(payload["scale"]),
            growth_tracker=int(payload.get("growth_tracker", 0)),
            total_steps=int(payload.get("total_steps", 0)),
            skipped_steps=int(payload.get("skipped_steps", 0)),
        )


class _DeviceFlag:
    """Truth value of a device-side non-finite flag, read (one sync) on first use."""

    def __init__(self, compute) -> None:
        self._compute = compute
        self._value: bool | None = None

    def __bool__(self) -> bool:
        if self._value is None:
            self._value = bool(self._compute())
        return self._value

    def __repr__(self) -> str:
        return f"_DeviceFlag({'unevaluated' if self._value is None else self._value})"


def _nonfinite_flag(params: Sequence[nn.Parameter], device: torch.device) -> torch.Tensor | None:
    grads = [p.grad for p in params if p.grad is not None]
    if not grads:
        return None
    segments = [(g, 0, int(g.numel()), 1.0) for g in grads]
    # The pass's partials stay on the gradients: an optimizer clipping the same,
    # unchanged gradients next (the engine's order) reads them instead of the gradients.
    # Gradients in host memory stream through the scaler's device.
    resident = next((g.device for g in grads if not is_host(g)), device)
    return gradient_norm_pass(segments, resident, max_norm=0.0, tag=True).nonfinite


def _apply_pending_unscale(grads: Sequence[torch.Tensor], device: torch.device) -> None:
    """Multiply each gradient that carries a deferred unscale factor by it in place,
    rounded to the gradient's dtype as ``grad.mul_`` rounds (``hbt_scale_inplace``),
    and drop the factor: the gradient is then what the in-place unscale leaves."""
    groups: dict[tuple[torch.device, torch.dtype, float], list[torch.Tensor]] = {}
    for g in grads:
        if g is None or not hasattr(g, PENDING_UNSCALE_ATTR):
            continue
        # the in-place scaling addresses numel consecutive elements: checked for every
        # gradient before any is scaled
        _native.require_dense(g, "grad_scaler.unscale_")
        if g.dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.float64):
            raise UnsupportedFeatureError(
                format_error("grad_scaler.unscale_", "gradients must be float64, float32, bfloat16 or float16",
                             observed=str(g.dtype))
            )
        resident = device if is_host(g) else g.device
        groups.setdefault((resident, g.dtype, float(getattr(g, PENDING_UNSCALE_ATTR))), []).append(g)
    for (resident, dtype, factor), batch in groups.items():
        scale_gradients(batch, dtype, factor, None, resident, "grad_scaler.hbt_scale_inplace")
        for g in batch:
            delattr(g, PENDING_UNSCALE_ATTR)


class GradScaler:
    """Loss scaler with a native unscale and overflow check (``grad_scaler.py:95-298``)."""

    def __init__(
        self,
        config: GradScalerConfig,
        group: GroupHandle,
        device: torch.device,
        *,
        recorder: Any = None,
        defer_unscale: bool = False,
    ) -> None:
        self._config = config
        self._group = group
        self._device = torch.device(device)
        self._recorder = recorder
        self._defer = defer_unscale
        self._state = GradScalerState(scale=config.init_scale if config.enabled else 1.0)
        self._unscaled = False
        self._skipped_on_last_step = False

    @property
    def enabled(self) -> bool:
        """Whether scaling is active."""
        return self._config.enabled

    @property
    def scale_value(self) -> float:
        """Current loss scale (1.0 when disabled)."""
        return self._state.scale if self._config.enabled else 1.0

    @property
    def state(self) -> GradScalerState:
        """Current scaler state."""
        return self._state

    def scale(self, loss: torch.Tensor) -> torch.Tensor:
        """Multiply the loss by the current scale (unchanged when disabled)."""
        if not self._config.enabled:
            return loss
        self._unscaled = False
        return loss * self._state.scale

    def unscale_(self, parameters: Iterable[nn.Parameter]) -> bool:
        """Divide gradients by the scale and report whether any is non-finite."""
        params = [p for p in parameters if p.grad is not None]
        if not self._config.enabled:
            return self._detect_non_finite(params)
        inverse = 1.0 / self._state.scale
        if self._defer:
            # A factor still pending from an earlier unscale_ (no step since) is applied
            # first, so two calls multiply twice, as two in-place multiplies do.
            _apply_pending_unscale([p.grad for p in params], self._device)
            # Float64 gradients are unscaled at once, in double: the norm and the update
            # read a deferred factor only through fp32 arithmetic.
            wide = [p for p in params if p.grad.dtype == torch.float64]
            for p in wide:
                setattr(p.grad, PENDING_UNSCALE_ATTR, inverse)
            _apply_pending_unscale([p.grad for p in wide], self._device)
            for p in params:
                if p.grad.dtype != torch.float64:
                    setattr(p.grad, PENDING_UNSCALE_ATTR, inverse)
            self._unscaled = True
            return _DeviceFlag(lambda: self._detect_non_finite(params))  # type: ignore[return-value]
        groups: dict[tuple[torch.device, torch.dtype], list[torch.Tensor]] = {}
        for p in params:
            if not is_host(p.grad):
                _native.require_device_tensor(p.grad, "grad_scaler.unscale_")
            _native.require_dense(p.grad, "grad_scaler.unscale_")
            if p.grad.dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.float64):
                raise UnsupportedFeatureError(
                    format_error("grad_scaler.unscale_", "gradients must be float64, float32, bfloat16 or float16",
                                 observed=str(p.grad.dtype))
                )
            # a gradient in host memory streams through the scaler's device
            device = self._device if is_host(p.grad) else p.grad.device
            groups.setdefault((device, p.grad.dtype), []).append(p.grad)
        for (device, dtype), grads in groups.items():
            # the unscale and the norm partials of its result in one pass; the check
            # below and the optimizer's clip take the norm from those partials
            unscale_with_partials(grads, dtype, inverse, device, "grad_scaler.hbt_scale_inplace_sqnorm")
        self._unscaled = True
        return self._detect_non_finite(params)

    def _detect_non_finite(
        self, parameters: Sequence[nn.Parameter], optimizer: Any = None
    ) -> bool:
        """Whether any gradient element is inf or NaN (one device flag, one sync)."""
        flag = None
        if optimizer is not None and hasattr(optimizer, "last_nonfinite_flag"):
            covered = {id(p) for p in getattr(optimizer, "parameters", ()) if p.grad is not None}
            if covered == {id(p) for p in parameters}:
                flag = optimizer.last_nonfinite_flag()
        if flag is None:
            flag = _nonfinite_flag(parameters, self._device)
        if flag is None:
            return False
        return bool(int(flag.item()) != 0)

    def step(
        self,
        optimizer: Any,
        parameters: Iterable[nn.Parameter],
        *,
        already_unscaled: bool = False,
    ) -> bool:
        """Step the optimizer unless a gradient is non-finite (``grad_scaler.py:202-241``)."""
        params = list(parameters)
        if already_unscaled or self._unscaled:
            found = self._detect_non_finite([p for p in params if p.grad is not None], optimizer)
        else:
            found = bool(self.unscale_(params))
        if not isinstance(optimizer, ShardedOptimizer):
            # Only ShardedOptimizer applies a deferred factor while it reads the gradient;
            # any other optimizer (the reference accepts a plain torch.optim.Optimizer)
            # gets gradients that are already unscaled.
            _apply_pending_unscale([p.grad for p in params], self._device)
        self._state.total_steps += 1
        self._skipped_on_last_step = found
        if found:
            # The reference has already unscaled and clipped .grad in place when it skips
            # (grad_scaler.py:181-186, sharded_optimizer.py:333-337); an optimizer that
            # keeps those semantics but defers the multiplies to its step applies them now.
            if getattr(optimizer, "clips_in_place", False):
                optimizer.materialize_pending()
            self._state.skipped_steps += 1
            # The reference logs every skipped step (grad_scaler.py:229-236).
            _LOGGER.warning(
                "non-finite gradient detected; skipping optimizer step %d and reducing the loss scale from %.1f",
                self._state.total_steps,
                self._state.scale,
            )
            return False
        optimizer.step()
        return True

    def update(self, *, found_non_finite: bool | None = None) -> float:
        """Grow or back off the scale (``grad_scaler.py:243-269``)."""
        if not self._config.enabled:
            return 1.0
        overflowed = found_non_finite if found_non_finite is not None else self._skipped_on_last_step
        if overflowed:
            self._state.scale = max(self._state.scale * self._config.backoff_factor, 1.0)
            self._state.growth_tracker = 0
        else:
            self._state.growth_tracker += 1
            if self._state.growth_tracker >= self._config.growth_interval:
                self._state.scale = min(
                    self._state.scale * self._config.growth_factor, self._config.max_scale
                )
                self._state.growth_tracker = 0
        self._unscaled = False
        return self._state.scale

    @property
    def last_step_skipped(self) -> bool:
        """True when the last :meth:`step` found a non-finite gradient and did not update."""
        return self._skipped_on_last_step

    def state_dict(self) -> dict[str, float]:
        """Scaler state for checkpointing."""
        return self._state.as_dict()

    def load_state_dict(self, payload: dict[str, Any]) -> None:
        """Restore :meth:`state_dict` output."""
        self._state = GradScalerState.from_dict(payload)
        self._unscaled = False

    def __repr__(self) -> str:
        return (
            f"GradScaler(enabled={self._config.enabled}, scale={self.scale_value}, "
            f"skipped={self._state.skipped_steps}/{self._state.total_steps})"
        )
