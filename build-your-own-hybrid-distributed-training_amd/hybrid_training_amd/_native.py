"""ctypes binding of ``libhbt.so`` and the host-side plumbing around it.

This is the only module that touches the C ABI declared in ``include/hbt.h``.  It
loads the library that sits next to this file, checks its ABI version, declares
every entry point's signature, turns non-zero status codes into
:class:`~hybrid_training_amd.errors.NativeKernelError`, and builds the interval
tables the gather-copy kernel consumes.

There is no fallback: when the library is missing, or a tensor is not on a HIP
device, the call raises.  Pointers come from ``Tensor.data_ptr()`` and the stream
from torch's current stream on the tensor's device, so every kernel is ordered
with the caller's other work on that stream.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from collections import OrderedDict
from collections.abc import Iterable, Sequence
from contextvars import ContextVar
from typing import Any

import torch
from torch.autograd.graph import increment_version

from .errors import NativeKernelError, ShardingError, UnsupportedFeatureError, format_error

__all__ = [
    "ABI_VERSION",
    "ACCUMULATE_ASSIGN",
    "COPY_ALIGNED",
    "COPY_HINTS",
    "COPY_CONVERSIONS",
    "OPTIMIZER_DTYPES",
    "STEP_SLOT_BYTES",
    "STEP_WRITE_GRAD",
    "COPY_OP_COPY",
    "COPY_OP_DIVIDE",
    "SGD_FIRST_STEP",
    "SGD_MOMENTUM",
    "SGD_NESTEROV",
    "SGD_WEIGHT_DECAY",
    "CopyPlan",
    "DTYPE_BF16",
    "DTYPE_F16",
    "DTYPE_F32",
    "DTYPE_F64",
    "EXPORTED_SYMBOLS",
    "GraphRecording",
    "MAX_LOCAL_RANKS",
    "MAX_TENSORS_PER_LAUNCH",
    "PIECES_PER_NORM_CHUNK",
    "check",
    "contiguous_source",
    "dtype_code",
    "graph_recording",
    "library",
    "library_path",
    "require_dense",
    "require_device_tensor",
    "stream_of",
]

ABI_VERSION = 18
MAX_TENSORS_PER_LAUNCH = 16
MAX_LOCAL_RANKS = 64
#: Doubles of working storage hbt_scale_inplace_sqnorm takes per partial for 2-byte gradients.
PIECES_PER_NORM_CHUNK = 128

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_F64 = 3

COPY_OP_COPY = 0
COPY_OP_DIVIDE = 1
COPY_ALIGNED = 1
COPY_HINTS = 2
#: Chunks per entry of a copy plan's hint table (HBT_COPY_HINTS).
COPY_HINT_STRIDE = 256
ACCUMULATE_ASSIGN = 1
_CODE_BYTES = {DTYPE_F32: 4, DTYPE_BF16: 2, DTYPE_F16: 2, DTYPE_F64: 8}

_FLOATS = (torch.float64, torch.float32, torch.bfloat16, torch.float16)
#: Dtype pairs ``hbt_copy_intervals`` converts between (same-dtype copies are bit copies):
#: every ordered pair of float64, float32, bfloat16 and float16, as ``Tensor.to`` converts.
COPY_CONVERSIONS = frozenset((a, b) for a in _FLOATS for b in _FLOATS if a != b)
SGD_MOMENTUM = 1
SGD_FIRST_STEP = 2
SGD_NESTEROV = 4
SGD_WEIGHT_DECAY = 8
#: hbt_adamw_step / hbt_sgd_step flag: store the unscaled, clipped gradient back.
STEP_WRITE_GRAD = 16
#: Bytes of device memory one step-scalar slot occupies (HBT_STEP_SLOT_BYTES).
STEP_SLOT_BYTES = 128
#: (parameter, gradient) dtype pairs the optimizer kernels update.
OPTIMIZER_DTYPES = frozenset({
    (torch.float32, torch.float32), (torch.float32, torch.bfloat16),
    (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
    (torch.float64, torch.float64),
})

_c_void_p = ctypes.c_void_p
_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_c_f64 = ctypes.c_double
_ptr_array = ctypes.POINTER(ctypes.c_void_p)
_i64_array = ctypes.POINTER(ctypes.c_int64)
_f64_array = ctypes.POINTER(ctypes.c_double)

#: Every entry point of include/hbt.h with its (restype, argtypes).
EXPORTED_SYMBOLS: dict[str, tuple[object, tuple[object, ...]]] = {
    "hbt_last_error": (ctypes.c_char_p, ()),
    "hbt_abi_version": (_c_i32, ()),
    "hbt_symbol_count": (_c_i32, ()),
    "hbt_grid_slices": (_c_i64, (_c_i64, _c_i32, _i64_array, _i64_array, _c_i64)),
    "hbt_adamw_step": (
        _c_i32,
        (
            _ptr_array, _ptr_array, _ptr_array, _ptr_array, _i64_array, _c_i32, _c_i32, _c_i32,
            _c_f32, _c_void_p, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32,
            _c_i32, _c_void_p,
        ),
    ),
    "hbt_sgd_step": (
        _c_i32,
        (
            _ptr_array, _ptr_array, _ptr_array, _i64_array, _c_i32, _c_i32, _c_i32, _c_f32, _c_void_p,
            _c_f32, _c_f32, _c_f32, _c_f32, _c_i32, _c_void_p,
        ),
    ),
    "hbt_norm_partials_count": (_c_i64, (_i64_array, _c_i32, _c_i32)),
    "hbt_grad_sqnorm_partials": (
        _c_i32,
        (_ptr_array, _i64_array, _f64_array, _c_i32, _c_i32, _c_f32, _c_void_p, _c_void_p),
    ),
    "hbt_grad_norm_finalize": (
        _c_i32,
        (_c_void_p, _c_i64, _c_f64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p),
    ),
    "hbt_grad_norm_noalloc": (
        _c_i32,
        (_ptr_array, _i64_array, _f64_array, _c_i32, _c_i32, _c_f32, _c_f64, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p),
    ),
    "hbt_copy_chunk_elems": (_c_i64, (_c_i32, _c_i32)),
    "hbt_copy_intervals": (
        _c_i32,
        (_c_void_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_f32, _c_i32, _c_void_p),
    ),
    "hbt_grad_local_share": (
        _c_i32,
        (_ptr_array, _c_i32, _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _c_f32, _c_i32, _c_void_p, _c_void_p),
    ),
    "hbt_grad_local_share_sqnorm": (
        _c_i32,
        (_ptr_array, _c_i32, _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _c_f32, _c_i32, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p),
    ),
    "hbt_grad_local_share_accumulated": (
        _c_i32,
        (_ptr_array, _ptr_array, _c_i32, _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _c_f32, _c_i32, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p),
    ),
    "hbt_scale_inplace": (
        _c_i32,
        (_ptr_array, _i64_array, _c_i32, _c_i32, _c_f32, _c_void_p, _c_void_p),
    ),
    "hbt_scale_inplace_sqnorm": (
        _c_i32,
        (_ptr_array, _i64_array, _c_i32, _c_i32, _c_f32, _c_void_p, _c_void_p, _c_void_p),
    ),
    "hbt_grad_accumulate": (
        _c_i32,
        (_ptr_array, _ptr_array, _i64_array, _c_i32, _c_i32, _c_i32, _c_i32, _c_void_p),
    ),
    "hbt_adamw_step_f64": (
        _c_i32,
        (
            _ptr_array, _ptr_array, _ptr_array, _ptr_array, _i64_array, _c_i32, _c_f64, _c_void_p,
            _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_i32, _c_void_p,
        ),
    ),
    "hbt_sgd_step_f64": (
        _c_i32,
        (
            _ptr_array, _ptr_array, _ptr_array, _i64_array, _c_i32, _c_f64, _c_void_p,
            _c_f64, _c_f64, _c_f64, _c_f64, _c_i32, _c_void_p,
        ),
    ),
    "hbt_scale_inplace_f64": (
        _c_i32,
        (_ptr_array, _i64_array, _c_i32, _c_f64, _c_void_p, _c_void_p),
    ),
    "hbt_adamw_step_slot": (
        _c_i32,
        (
            _ptr_array, _ptr_array, _ptr_array, _ptr_array, _i64_array, _c_i32, _c_i32, _c_i32,
            _c_f32, _c_void_p, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32,
            _c_void_p, _c_i32, _c_void_p,
        ),
    ),
    "hbt_adamw_write_scalars": (
        _c_i32,
        (_c_void_p, _c_i32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_void_p),
    ),
    "hbt_sgd_step_slot": (
        _c_i32,
        (
            _ptr_array, _ptr_array, _ptr_array, _i64_array, _c_i32, _c_i32, _c_i32, _c_f32, _c_void_p,
            _c_f32, _c_f32, _c_f32, _c_f32, _c_void_p, _c_i32, _c_void_p,
        ),
    ),
    "hbt_sgd_write_scalars": (
        _c_i32,
        (_c_void_p, _c_i32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_i32, _c_void_p),
    ),
    "hbt_adamw_step_f64_slot": (
        _c_i32,
        (
            _ptr_array, _ptr_array, _ptr_array, _ptr_array, _i64_array, _c_i32, _c_f64, _c_void_p,
            _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_void_p, _c_i32, _c_void_p,
        ),
    ),
    "hbt_adamw_write_scalars_f64": (
        _c_i32,
        (_c_void_p, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_void_p),
    ),
    "hbt_sgd_step_f64_slot": (
        _c_i32,
        (
            _ptr_array, _ptr_array, _ptr_array, _i64_array, _c_i32, _c_f64, _c_void_p,
            _c_f64, _c_f64, _c_f64, _c_f64, _c_void_p, _c_i32, _c_void_p,
        ),
    ),
    "hbt_sgd_write_scalars_f64": (
        _c_i32,
        (_c_void_p, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_i32, _c_void_p),
    ),
    "hbt_adamw_scalar_record": (
        _c_i32,
        (_c_void_p, _c_i32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32),
    ),
    "hbt_sgd_scalar_record": (_c_i32, (_c_void_p, _c_i32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_i32)),
    "hbt_adamw_scalar_record_f64": (
        _c_i32,
        (_c_void_p, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64),
    ),
    "hbt_sgd_scalar_record_f64": (_c_i32, (_c_void_p, _c_f64, _c_f64, _c_f64, _c_f64, _c_f64, _c_i32)),
    "hbt_write_words": (_c_i32, (_c_void_p, ctypes.POINTER(ctypes.c_uint32), _c_i64, _c_void_p)),
}

_LOCK = threading.Lock()
# Guards the copy-table cache for callers that run copy plans from several host threads.
_TABLE_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None

# Device copies of interval tables, keyed by their exact content.  A table is a pure
# function of its rows (addresses, lengths, chunk prefix), so an entry stays valid
# even after the tensors it was built for are freed; reuse skips the host-to-device
# upload, which for a few hundred rows costs more than moving a GB on the device.
_TABLE_CACHE: "OrderedDict[tuple, tuple[torch.Tensor, int, bool, bool]]" = OrderedDict()
_TABLE_CACHE_SIZE = 256


class GraphRecording:
    """What a :class:`~hybrid_training_amd.graphs.StepGraph` collects while it records:
    the optimizer launches whose scalars each replay rewrites (``steps``, objects whose
    ``prepare()`` checks the recorded launch and returns the action that rewrites them)
    and the device tables recorded launches read (``tables``), which must live as long
    as the graph.

    The step-scalar slots come from one slab allocated before the capture starts, not
    from the graph's private pool: the host writes a slot before each replay and the
    replay reads it, while a block of the private pool may also belong to a temporary
    that an earlier recorded launch writes during the same replay.  Each slot has a
    host record of the same size (:meth:`record_address`): before a replay every
    recorded step formats its scalars into its record, and :meth:`write_slots` copies
    all of them into the slab with one launch per 256 words.
    """

    #: Step-scalar slots one recording can hand out.
    MAX_SLOTS = 256

    def __init__(self, device: torch.device) -> None:
        self.steps: list[Any] = []
        self.tables: list[torch.Tensor] = []
        self._device = device
        self._slab = torch.zeros(self.MAX_SLOTS * STEP_SLOT_BYTES // 8, dtype=torch.float64, device=device)
        self._records = (ctypes.c_uint32 * (self.MAX_SLOTS * STEP_SLOT_BYTES // 4))()
        self._used = 0

    def record_address(self, slot: torch.Tensor) -> int:
        """Host address of the record that :meth:`write_slots` copies into ``slot``."""
        offset = slot.data_ptr() - self._slab.data_ptr()
        if not 0 <= offset < self._used * STEP_SLOT_BYTES or offset % STEP_SLOT_BYTES:
            raise ValueError("not a slot of this recording")
        return ctypes.addressof(self._records) + offset

    def write_slots(self) -> None:
        """Copy every handed-out slot's host record into the slab, on the current stream."""
        if self._used:
            check(library().hbt_write_words(self._slab.data_ptr(), self._records, self._used * STEP_SLOT_BYTES // 4,
                                            stream_of(self._device)),
                  "native.GraphRecording.write_slots")

    def new_slot(self) -> torch.Tensor:
        """``STEP_SLOT_BYTES`` of device memory outside the graph's pool."""
        if self._used == self.MAX_SLOTS:
            raise UnsupportedFeatureError(
                format_error("native.GraphRecording", "the step function launches more optimizer batches than "
                             "one recording holds slots for", expected=f"at most {self.MAX_SLOTS}")
            )
        per = STEP_SLOT_BYTES // 8
        slot = self._slab[self._used * per : (self._used + 1) * per]
        self._used += 1
        return slot


_RECORDING: ContextVar[GraphRecording | None] = ContextVar("hbt_graph_recording", default=None)


def graph_recording() -> GraphRecording | None:
    """The recording in progress, or ``None`` when launches run eagerly.

    Raises:
        UnsupportedFeatureError: if torch's current stream is being captured into a
            HIP graph without a recording (a bare ``torch.cuda.graph``): a recorded
            step would replay the scalars and tables of its recording forever.
    """
    recording = _RECORDING.get()
    # No capture can be in progress before torch has initialised the device; the raw
    # query skips torch.cuda.is_available(), which reads the environment on every call.
    if recording is None and torch.cuda.is_initialized() and _IS_CAPTURING is not None and _IS_CAPTURING():
        raise UnsupportedFeatureError(
            format_error("native.graph_recording",
                         "this work is being captured into a HIP graph outside hybrid_training_amd.StepGraph, "
                         "whose replays would repeat the recorded step scalars and copy tables",
                         resolution="record the step with hybrid_training_amd.StepGraph")
        )
    return recording


def set_graph_recording(recording: GraphRecording | None):
    """Make ``recording`` the current one; returns the token that restores the previous."""
    return _RECORDING.set(recording)


def reset_graph_recording(token) -> None:
    _RECORDING.reset(token)


def write_words(device: torch.device, dst: torch.Tensor, words: Sequence[int]) -> None:
    """Write 32-bit ``words`` into the dense device tensor ``dst`` (at least as many bytes)
    by launches that carry them as arguments (``hbt_write_words``) on the current stream."""
    require_device_tensor(dst, "native.write_words")
    if len(words) * 4 > dst.numel() * dst.element_size():
        raise ValueError("more words than the destination holds")
    host = (ctypes.c_uint32 * max(1, len(words)))(*words)
    with torch.cuda.device(device):
        check(library().hbt_write_words(dst.data_ptr(), host, len(words), stream_of(device)), "native.write_words")


def release_tables() -> None:
    """Drop every cached device table of a copy plan (rebuilt on the next use)."""
    with _TABLE_LOCK:
        _TABLE_CACHE.clear()


def library_path() -> str:
    """Absolute path of ``libhbt.so`` inside this package."""
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhbt.so")


def library() -> ctypes.CDLL:
    """Load (once) and return ``libhbt.so`` with every signature declared.

    Raises:
        NativeKernelError: if the file is absent, fails to load, exports the wrong
            symbol set, or reports a different ABI version.
    """
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not os.path.exists(path):
            raise NativeKernelError(
                format_error(
                    "native.library",
                    "libhbt.so has not been built; there is no non-native fallback",
                    expected=path,
                    observed="missing",
                    resolution="run __graft_entry__.build() or `make -C <package>/csrc`",
                )
            )
        try:
            lib = ctypes.CDLL(path)
        except OSError as exc:
            raise NativeKernelError(
                format_error("native.library", f"cannot load libhbt.so: {exc}", observed=path)
            ) from exc
        for name, (restype, argtypes) in EXPORTED_SYMBOLS.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as exc:
                raise NativeKernelError(
                    format_error("native.library", "missing entry point", expected=name, observed=path)
                ) from exc
            fn.restype = restype
            fn.argtypes = list(argtypes)
        version = lib.hbt_abi_version()
        if version != ABI_VERSION:
            raise NativeKernelError(
                format_error(
                    "native.library",
                    "libhbt.so was built from a different ABI",
                    expected=ABI_VERSION,
                    observed=version,
                    resolution="rebuild the library",
                )
            )
        if lib.hbt_symbol_count() != len(EXPORTED_SYMBOLS):
            raise NativeKernelError(
                format_error(
                    "native.library",
                    "the library and the binding disagree on the entry-point count",
                    expected=len(EXPORTED_SYMBOLS),
                    observed=lib.hbt_symbol_count(),
                    resolution="rebuild the library",
                )
            )
        _LIB = lib
        return lib


def check(status: int, operation: str) -> None:
    """Raise :class:`NativeKernelError` for a non-zero status from ``libhbt.so``."""
    if status != 0:
        message = library().hbt_last_error() or b""
        raise NativeKernelError(
            format_error(operation, message.decode(errors="replace") or "native call failed",
                         observed=f"status {status}")
        )


_DTYPE_CODES = {
    torch.float32: DTYPE_F32,
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_F16,
    torch.float64: DTYPE_F64,
}


def dtype_code(dtype: torch.dtype) -> int:
    """ABI code of a floating dtype."""
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise UnsupportedFeatureError(
            format_error(
                "native.dtype_code",
                "dtype not handled by the HIP kernels",
                expected=sorted(str(d) for d in _DTYPE_CODES),
                observed=str(dtype),
            )
        ) from exc


def require_device_tensor(tensor: torch.Tensor, operation: str) -> None:
    """Refuse host tensors: every data path here runs on the HIP device."""
    if tensor.device.type != "cuda":
        raise UnsupportedFeatureError(
            format_error(
                operation,
                "hybrid_training_amd runs the hot path only as HIP kernels, so tensors must live "
                "on a HIP device",
                expected="device type 'cuda' (HIP)",
                observed=str(tensor.device),
                resolution="move the tensors to the GPU first",
            )
        )


def require_dense(tensor: torch.Tensor, operation: str) -> None:
    """Refuse a tensor whose elements are not the ``numel`` consecutive ones from its
    address: the element-wise kernels address exactly that range."""
    if not tensor.is_contiguous():
        raise ShardingError(
            format_error(operation, "gradients must be dense", expected="a contiguous tensor",
                         observed=f"shape {tuple(tensor.shape)}, strides {tuple(tensor.stride())}",
                         resolution="pass a contiguous gradient (for example grad.contiguous())")
        )


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_IS_CAPTURING = getattr(torch._C, "_cuda_isCurrentStreamCapturing", None)
_RAW_DEVICE = getattr(torch._C, "_cuda_getDevice", None)
_NO_GUARD = contextlib.nullcontext()


def _current_device() -> int:
    """torch's current device index; once torch has initialised the device, read without
    its lazy-initialisation check (every launch's host path asks)."""
    if _RAW_DEVICE is not None and torch.cuda.is_initialized():
        return int(_RAW_DEVICE())
    return torch.cuda.current_device()


def device_guard(device: torch.device):
    """``torch.cuda.device(device)``, or a context that does nothing when ``device`` is
    already the current one (the usual case: a guard costs about a microsecond of host
    time, and every launch's host path takes one)."""
    if isinstance(device, torch.device) and device.type == "cuda" and (
            device.index is None or device.index == _current_device()):
        return _NO_GUARD
    return torch.cuda.device(device)


def stream_of(device: torch.device) -> int:
    """Raw ``hipStream_t`` of torch's current stream on ``device`` (read without building
    a ``torch.cuda.Stream`` object: this is on every launch's host path)."""
    if _RAW_STREAM is not None:
        index = device.index if isinstance(device, torch.device) else torch.device(device).index
        return int(_RAW_STREAM(_current_device() if index is None else index))
    return int(torch.cuda.current_stream(device).cuda_stream)


def contiguous_source(tensor: torch.Tensor) -> torch.Tensor:
    """``tensor`` when it is dense, else a dense copy (the reference's ``reshape(-1)``)."""
    return tensor if tensor.is_contiguous() else tensor.contiguous()


def pointer_array(values: Sequence[int]) -> ctypes.Array:
    """ctypes ``void*[]`` holding device addresses."""
    return (ctypes.c_void_p * max(1, len(values)))(*values)


def int64_array(values: Sequence[int]) -> ctypes.Array:
    """ctypes ``int64_t[]``."""
    return (ctypes.c_int64 * max(1, len(values)))(*values)


def double_array(values: Sequence[float]) -> ctypes.Array:
    """ctypes ``double[]``."""
    return (ctypes.c_double * max(1, len(values)))(*values)


_CHUNKS: dict[tuple[int, int], int] = {}


def _copy_chunk(lib: ctypes.CDLL, src_code: int, dst_code: int) -> int:
    """Elements per copy-kernel chunk for a dtype pair."""
    key = (src_code, dst_code)
    chunk = _CHUNKS.get(key)
    if chunk is None:
        chunk = int(lib.hbt_copy_chunk_elems(src_code, dst_code))
        if chunk <= 0:
            raise UnsupportedFeatureError(
                format_error("native.CopyPlan", "the copy kernel does not move this dtype pair",
                             observed=key)
            )
        _CHUNKS[key] = chunk
    return chunk


def plan_table(rows: Sequence[tuple[int, int, int]], chunk: int, scale: int = 1) -> tuple[list[int], int]:
    """The flat ``{src, dst, numel, first_chunk}`` records of a plan and its chunk count.

    ``scale`` multiplies every numel (2 when 8-byte elements travel as dword pairs).
    """
    flat: list[int] = []
    first = 0
    for src_addr, dst_addr, n in rows:
        n_units = n * scale
        flat.extend((src_addr, dst_addr, n_units, first))
        first += -(-n_units // chunk)
    return flat, first


def plan_hints(first_chunks: Sequence[int], total_chunks: int) -> list[int]:
    """The ``HBT_COPY_HINTS`` table of a plan: for every ``COPY_HINT_STRIDE``-th chunk, the
    index of the record that owns it (the last record starting at or before it)."""
    import numpy as np

    starts = np.asarray(first_chunks, dtype=np.int64)
    probes = np.arange(0, total_chunks, COPY_HINT_STRIDE, dtype=np.int64)
    return (np.searchsorted(starts, probes, side="right") - 1).tolist()


def plan_is_aligned(rows: Sequence[tuple[int, int, int]], src_code: int, dst_code: int) -> bool:
    """Whether a plan qualifies for ``HBT_COPY_ALIGNED``: every destination on a 16-byte
    boundary and every source (0 for a zero fill) on the source width of one 16-byte
    unit, ``16 * S / max(S, D)`` bytes for S- and D-byte elements."""
    src_bytes, dst_bytes = _CODE_BYTES[src_code], _CODE_BYTES[dst_code]
    src_align = 16 * src_bytes // max(src_bytes, dst_bytes)
    return all(dst_addr % 16 == 0 and src_addr % src_align == 0 for src_addr, dst_addr, _ in rows)


def _prepared_plan(
    device: torch.device, rows: tuple[tuple[int, int, int], ...], src_code: int, dst_code: int, scale: int
) -> tuple[torch.Tensor, int, bool, bool]:
    """(device table, total chunks, aligned, hinted) for a plan, built once per distinct plan
    and stream.  The table is uploaded on that stream, so later launches on it see it."""
    recording = graph_recording()
    stream = stream_of(device)
    key = (device, stream, src_code, dst_code, scale, rows)
    if recording is None:
        with _TABLE_LOCK:
            entry = _TABLE_CACHE.get(key)
            if entry is not None:
                _TABLE_CACHE.move_to_end(key)
                return entry
    chunk = _copy_chunk(library(), src_code, dst_code)
    flat, first = plan_table(rows, chunk, scale)
    aligned = plan_is_aligned(rows, src_code, dst_code)
    # Plans of several records carry the hint table after their records.
    hinted = len(rows) > 1
    if hinted:
        flat = flat + plan_hints(flat[3::4], first)
    if recording is not None:
        # Inside a graph recording the table is written by launches that carry it in
        # their arguments, so every replay rewrites it from the recorded words; the
        # graph owns it (a host-to-device copy from pageable memory cannot be recorded).
        table = torch.empty(len(flat), dtype=torch.int64, device=device)
        words = []
        for value in flat:
            words.extend((value & 0xFFFFFFFF, (value >> 32) & 0xFFFFFFFF))
        write_words(device, table, words)
        recording.tables.append(table)
        return table, first, aligned, hinted
    host = torch.tensor(flat, dtype=torch.int64).pin_memory()
    with torch.cuda.device(device):
        table = host.to(device, non_blocking=True)
    entry = (table, first, aligned, hinted)
    with _TABLE_LOCK:
        _TABLE_CACHE[key] = entry
        if len(_TABLE_CACHE) > _TABLE_CACHE_SIZE:
            _TABLE_CACHE.popitem(last=False)
    return entry


def bump_versions(tensors: Iterable[torch.Tensor]) -> None:
    """Advance the autograd version counter of every tensor a kernel wrote in place
    (inference tensors carry none and are skipped).

    Writes that bypass the counter, such as ones made through ``tensor.data`` or by
    foreign code holding a raw pointer, are not seen: a gradient's cached norm partials
    (keyed by address and version) then describe the old values.
    """
    written = [t for t in tensors if not t.is_inference()]
    if written:
        increment_version(written)


class CopyPlan:
    """Interval table for one ``hbt_copy_intervals`` launch.

    Each :meth:`add` appends ``n`` elements from ``src[src_offset:]`` to
    ``dst[dst_offset:]`` (offsets in elements of each tensor's own dtype, counted
    from the tensor's first element); :meth:`add_zero` appends a zero fill.  All
    records of one plan share a source dtype, a destination dtype and an op.  Ranges
    must not overlap between records.
    """

    def __init__(self, device: torch.device) -> None:
        self.device = torch.device(device)
        self._rows: list[tuple[int, int, int]] = []
        # The tensors the rows address, held for the plan's lifetime.  A row records
        # only addresses: a temporary the caller made for it (a dense or device copy)
        # and dropped before run() would hand its memory to the next allocation on the
        # stream, this plan's own table among them, before the kernel reads it.
        self._keep: list[torch.Tensor] = []
        # The tensors the plan writes: run() bumps their autograd version counters, as the
        # in-place copy_ it replaces would, so anything keyed on a version (a gradient's
        # cached norm partials, autograd's saved-tensor checks) sees the change.
        self._dests: dict[int, torch.Tensor] = {}

    def __len__(self) -> int:
        return len(self._rows)

    @classmethod
    def from_rows(cls, device: torch.device, rows: list[tuple[int, int, int]]) -> "CopyPlan":
        """A plan over rows ``(source address or 0 for a zero fill, destination address, n)``.

        For callers that have already checked every address against a dense device
        tensor of the plan's dtypes and every extent against that tensor's end, and
        that keep those tensors alive until :meth:`run` has returned, and that bump the
        version counters of the tensors written (:func:`bump_versions`).
        """
        plan = cls(device)
        plan._rows = [row for row in rows if row[2] > 0]
        return plan

    def add(self, src: torch.Tensor, src_offset: int, dst: torch.Tensor, dst_offset: int, n: int) -> None:
        """Queue ``dst[dst_offset : dst_offset + n] = src[src_offset : src_offset + n]``."""
        require_device_tensor(src, "native.CopyPlan")
        require_device_tensor(dst, "native.CopyPlan")
        if n < 0 or src_offset < 0 or dst_offset < 0:
            raise ValueError("negative copy extent")
        if src_offset + n > src.numel() or dst_offset + n > dst.numel():
            raise ValueError(
                f"copy of {n} elements runs past a tensor end "
                f"(src {src_offset}+{n}>{src.numel()} or dst {dst_offset}+{n}>{dst.numel()})"
            )
        if not (src.is_contiguous() and dst.is_contiguous()):
            raise ValueError("copy plans address dense tensors only")
        if n == 0:
            return
        self._keep.append(src)
        self._dests[id(dst)] = dst
        self._rows.append(
            (
                src.data_ptr() + src_offset * src.element_size(),
                dst.data_ptr() + dst_offset * dst.element_size(),
                n,
            )
        )

    def add_zero(self, dst: torch.Tensor, dst_offset: int, n: int) -> None:
        """Queue ``dst[dst_offset : dst_offset + n] = 0``."""
        require_device_tensor(dst, "native.CopyPlan")
        if n < 0 or dst_offset < 0 or dst_offset + n > dst.numel():
            raise ValueError("zero fill runs past the tensor end")
        if not dst.is_contiguous():
            raise ValueError("copy plans address dense tensors only")
        if n == 0:
            return
        self._dests[id(dst)] = dst
        self._rows.append((0, dst.data_ptr() + dst_offset * dst.element_size(), n))

    def run(
        self,
        *,
        src_dtype: torch.dtype,
        dst_dtype: torch.dtype,
        op: int = COPY_OP_COPY,
        divisor: float = 1.0,
    ) -> None:
        """Launch the copy on the current stream of the plan's device."""
        if not self._rows:
            return
        src_code = dtype_code(src_dtype)
        dst_code = dtype_code(dst_dtype)
        scale = 1
        if src_dtype == dst_dtype and op == COPY_OP_COPY and src_code == DTYPE_F64:
            # An 8-byte element moves as two dwords.
            src_code = dst_code = DTYPE_F32
            scale = 2
        lib = library()
        table, first, aligned, hinted = _prepared_plan(self.device, tuple(self._rows), src_code, dst_code, scale)
        with device_guard(self.device):
            status = lib.hbt_copy_intervals(
                table.data_ptr(),
                len(self._rows),
                first,
                src_code,
                dst_code,
                op,
                float(divisor),
                (COPY_ALIGNED if aligned else 0) | (COPY_HINTS if hinted else 0),
                stream_of(self.device),
            )
        check(status, "native.hbt_copy_intervals")
        bump_versions(self._dests.values())
