"""Configuration knobs of the data-parallel hot path.

Only the dataclasses the hot path reads are kept: optimizer hyper-parameters,
the DDP bucket knobs, the FSDP flat-parameter knobs, the loss scaler and the
mixed-precision policy.  Field names, defaults and validation follow
``config.py:361-491``, ``:533-656`` and ``:822-878`` of the reference so that a
configuration built for the reference builds here unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .errors import ConfigurationError, format_error

__all__ = [
    "DDPConfig",
    "FSDPConfig",
    "GradScalerConfig",
    "MixedPrecisionConfig",
    "OptimizerConfig",
    "resolve_dtype",
]

_DTYPE_NAMES: dict[str, torch.dtype] = {
    "float32": torch.float32,
    "fp32": torch.float32,
    "float64": torch.float64,
    "fp64": torch.float64,
    "float16": torch.float16,
    "fp16": torch.float16,
    "half": torch.float16,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
}


def resolve_dtype(name: str | torch.dtype) -> torch.dtype:
    """``torch.dtype`` for a dtype or one of the accepted names (``config.py:65-92``)."""
    if isinstance(name, torch.dtype):
        return name
    key = str(name).lower().replace("torch.", "")
    if key not in _DTYPE_NAMES:
        raise ConfigurationError(
            format_error(
                "config.resolve_dtype",
                "unknown dtype name",
                expected=sorted(_DTYPE_NAMES),
                observed=name,
                resolution="name a float dtype as listed (case and a 'torch.' prefix are ignored)",
            )
        )
    return _DTYPE_NAMES[key]


def _fail(owner: str, problem: str, expected: object, observed: object, fix: str) -> None:
    raise ConfigurationError(
        format_error(f"config.{owner}", problem, expected=expected, observed=observed, resolution=fix)
    )


@dataclass(frozen=True)
class DDPConfig:
    """Gradient-bucketing knobs (``config.py:361-418``)."""

    bucket_cap_mb: float = 25.0
    broadcast_buffers: bool = True
    find_unused_parameters: bool = False
    average_gradients: bool = True
    async_reduction: bool = True
    check_parameter_consistency: bool = True
    source_rank_in_group: int = 0

    def __post_init__(self) -> None:
        if self.bucket_cap_mb <= 0:
            _fail("DDPConfig", "bucket_cap_mb must be positive", "> 0", self.bucket_cap_mb,
                  "buckets hold at least one gradient, so the cap must be above zero")
        if self.source_rank_in_group < 0:
            _fail("DDPConfig", "source_rank_in_group must be non-negative", ">= 0",
                  self.source_rank_in_group, "index the source rank inside its group, from 0")


@dataclass(frozen=True)
class FSDPConfig:
    """Flat-parameter knobs (``config.py:421-491``)."""

    reshard_after_forward: bool = True
    average_gradients: bool = True
    auto_wrap_min_num_params: int = 0
    cpu_offload_params: bool = False
    limit_all_gather_bytes: int = 0
    check_reduction_order: bool = False
    use_padding: bool = True

    def __post_init__(self) -> None:
        if self.auto_wrap_min_num_params < 0:
            _fail("FSDPConfig", "auto_wrap_min_num_params must be non-negative", ">= 0",
                  self.auto_wrap_min_num_params, "0 turns automatic wrapping off")
        if self.limit_all_gather_bytes < 0:
            _fail("FSDPConfig", "limit_all_gather_bytes must be non-negative", ">= 0",
                  self.limit_all_gather_bytes, "0 means no limit")
        if not self.use_padding:
            _fail(
                "FSDPConfig",
                "use_padding=False is not supported: every rank's shard must hold the same number "
                "of elements, and only a padded flat parameter splits that way for any size",
                True,
                False,
                "keep use_padding=True",
            )


@dataclass(frozen=True)
class GradScalerConfig:
    """Dynamic loss-scaling policy (``config.py:533-597``)."""

    enabled: bool = False
    init_scale: float = 65536.0
    growth_factor: float = 2.0
    backoff_factor: float = 0.5
    growth_interval: int = 2000
    max_scale: float = 2.0**24

    def __post_init__(self) -> None:
        if self.init_scale <= 0:
            _fail("GradScalerConfig", "init_scale must be positive", "> 0", self.init_scale,
                  "a power of two keeps the scaling exact; 2**16 is the usual start")
        if not self.growth_factor > 1.0:
            _fail("GradScalerConfig", "growth_factor must exceed 1", "> 1.0", self.growth_factor,
                  "2.0 doubles the scale after each clean interval")
        if not 0.0 < self.backoff_factor < 1.0:
            _fail("GradScalerConfig", "backoff_factor must lie in (0, 1)", "0 < x < 1",
                  self.backoff_factor, "0.5 halves the scale after an overflow")
        if self.growth_interval < 1:
            _fail("GradScalerConfig", "growth_interval must be at least 1", ">= 1",
                  self.growth_interval, "count clean steps between growths, e.g. 2000")


@dataclass(frozen=True)
class MixedPrecisionConfig:
    """Dtype policy of flat parameters and gradients (``config.py:600-656``)."""

    enabled: bool = False
    param_dtype: str = "bfloat16"
    reduce_dtype: str = "float32"
    buffer_dtype: str = "float32"
    master_dtype: str = "float32"
    scaler: GradScalerConfig = field(default_factory=GradScalerConfig)

    def __post_init__(self) -> None:
        for name in ("param_dtype", "reduce_dtype", "buffer_dtype", "master_dtype"):
            resolve_dtype(getattr(self, name))
        if self.enabled and self.scaler.enabled and resolve_dtype(self.param_dtype) is not torch.float16:
            _fail(
                "MixedPrecisionConfig",
                "loss scaling is only meaningful for float16 compute: a bfloat16 gradient has "
                "float32's 8-bit exponent and keeps small values that float16 flushes to zero",
                "float16",
                self.param_dtype,
                "compute in float16, or turn the scaler off",
            )

    @property
    def compute_dtype(self) -> torch.dtype:
        """Dtype of gathered parameters used for compute."""
        return resolve_dtype(self.param_dtype) if self.enabled else resolve_dtype(self.master_dtype)

    @property
    def gradient_reduce_dtype(self) -> torch.dtype:
        """Dtype gradients are reduced in."""
        return resolve_dtype(self.reduce_dtype) if self.enabled else resolve_dtype(self.master_dtype)


@dataclass(frozen=True)
class OptimizerConfig:
    """Optimizer hyper-parameters (``config.py:822-878``)."""

    name: str = "adamw"
    learning_rate: float = 1e-3
    weight_decay: float = 0.0
    betas: tuple[float, float] = (0.9, 0.999)
    eps: float = 1e-8
    momentum: float = 0.0
    cpu_offload_state: bool = False

    def __post_init__(self) -> None:
        if self.name not in {"adamw", "sgd"}:
            _fail("OptimizerConfig", "unknown optimizer", ["adamw", "sgd"], self.name,
                  "the step kernels implement AdamW and SGD")
        if self.learning_rate <= 0:
            _fail("OptimizerConfig", "learning_rate must be positive", "> 0", self.learning_rate,
                  "a step needs a learning rate above zero")
        betas = tuple(self.betas)
        if len(betas) != 2 or not all(0.0 <= b < 1.0 for b in betas):
            _fail("OptimizerConfig", "betas must be two values in [0, 1)",
                  "(b1, b2) with 0 <= b < 1", self.betas, "e.g. (0.9, 0.999)")
        object.__setattr__(self, "betas", betas)
