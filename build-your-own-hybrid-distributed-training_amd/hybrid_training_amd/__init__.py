"""MI355X-native data-parallel hot path of hybrid distributed training.

Drop-in replacements for the reference's flat-parameter, gradient-bucket,
sharded-optimizer, loss-scaler and checkpoint-interval objects, whose tensor work
runs in hand-written gfx950 HIP kernels reached through ``libhbt.so``'s C ABI
(``include/hbt.h``).  Importing the package does not load the library; the first
call that moves data does, and raises if it is missing.
"""

from __future__ import annotations

from .config import (
    DDPConfig,
    FSDPConfig,
    GradScalerConfig,
    MixedPrecisionConfig,
    OptimizerConfig,
    resolve_dtype,
)
from .errors import (
    CheckpointCorruptionError,
    CheckpointError,
    CheckpointVersionError,
    HybridTrainingError,
    IncompleteCheckpointError,
    NativeKernelError,
    ShardingError,
    UnsupportedFeatureError,
    format_error,
)
from .buckets import BucketedGradients, BucketLayout, GradientBucket, build_buckets
from .flat_param import (FlatParameter, FlatParamHandle, PieceLayout, ShardedTensorPiece, optimizer_parameter_layout,
                         reshard_state_dict_pieces)
from .grad_scaler import GradScaler, GradScalerState
from .graphs import StepGraph
from .groups import GroupHandle
from .manifest import (
    CheckpointManifest,
    FileRecord,
    ShardRecord,
    TensorRecord,
    checkpoint_directory_name,
    shard_filename,
    validate_shard_filename,
)
from .optim import (
    NormContribution,
    ShardedOptimizer,
    build_gradient_norm_contributions,
    build_inner_optimizer,
    distributed_gradient_norm,
)
from .reshard import DeviceShardCache, describe_reshard, load_flat_shard, read_tensor_range
from .checkpoint import (
    ShardFileCache,
    collect_flat_shard_payload,
    load_flat_shard_checkpoint,
    verify_files,
    write_checkpoint,
)
from .tensors import (
    FlatEntry,
    ShardRange,
    build_flat_layout,
    concat_shard_sizes,
    even_shard_ranges,
    flatten_dense_tensors,
    intersect_ranges,
    pad_flat_tensor,
    shard_range_for,
    unflatten_to_views,
)

__version__ = "0.1.0"


def _release_device_state() -> None:
    """Exit hook: settle the device before the C++ runtimes tear down.

    Python exit hooks run before the static destructors of torch and of the HIP runtime.
    By then a streamed pass may still have non-blocking copies in flight into pinned host
    memory, and this package still caches device objects: the staging streams, their
    events and buffers (``host_staging``) and the device tables of copy plans
    (``_native``).  Waiting for every device, dropping those caches and handing torch's
    cached device and pinned blocks back to the runtime here, while it is fully up, leaves
    the static destructors nothing of this package's to free in an unknown order.
    """
    import gc

    import torch

    from . import _native, host_staging

    if not torch.cuda.is_initialized():
        return
    for index in range(torch.cuda.device_count()):
        with torch.cuda.device(index):
            torch.cuda.synchronize()
    host_staging.release_streams()
    _native.release_tables()
    gc.collect()
    torch.cuda.empty_cache()
    if hasattr(torch._C, "_host_emptyCache"):
        torch._C._host_emptyCache()


import atexit as _atexit  # noqa: E402  (registered after torch's own hooks, so it runs first)

_atexit.register(_release_device_state)
