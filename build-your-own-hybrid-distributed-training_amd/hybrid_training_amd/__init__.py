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
