"""CPU oracle for the data-parallel hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` import this package: to check results, or to time
the reference's CPU arithmetic.
The product (``libhbt.so`` and ``hybrid_training_amd``) never imports it.

Each function restates the reference's algorithm for one piece of the path with
numpy, plain Python or the C restatement in ``hbt_oracle.c``, and cites the
reference lines it follows.  How each function is pinned (golden vectors from
the reference's tests, library routines, closed forms, brute force) is listed in
``PINNED_BY``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from collections.abc import Sequence

import numpy as np

__all__ = [
    "DTYPE_CODES",
    "PINNED_BY",
    "adamw_scalars",
    "adamw_step",
    "adamw_step_f64",
    "bucket_layout",
    "clip_multiplier",
    "clip_multiplier64",
    "even_shards",
    "f16_nan_rules",
    "f32_to_bf16",
    "flat_layout",
    "from_bits",
    "library",
    "local_share",
    "no_sync_accumulate",
    "pack_shard",
    "read_range",
    "round_to",
    "sgd_step",
    "sgd_step_f64",
    "sqnorm",
    "sqnorm_f64",
    "to_bits",
    "unpack_full",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libhbt_oracle.so")
_LIB: ctypes.CDLL | None = None

#: How each restatement is held to the reference (see tests/test_oracle_*.py).
PINNED_BY = {
    "flat_layout": "reference known answers: offsets 0/6/10 total 16 (test_tensor_utils.py:35-49); "
    "1857 params -> 929 pad 1 / 465 pad 3 (test_fsdp.py:373-399, README.md:106-107)",
    "even_shards": "reference known answers (test_tensor_utils.py:140-183) and the "
    "4-writer/3-reader intersection table (test_tensor_utils.py:219-230)",
    "pack_shard": "bitwise equality with torch.cat of reshape(-1) + zero padding + slicing "
    "(test_tensor_utils.py:51-61, test_fsdp.py:501-517)",
    "bucket_layout": "reverse-order/contiguity/exactly-once rules "
    "(test_single_process_components.py:145-178); GPT-2-small bucket counts",
    "clip_multiplier": "known answers: norm 6 -> clipped norm 1 (test_single_process_components.py:397-406)",
    "sqnorm": "math.fsum brute force; weighted known answer 1.25 "
    "(test_single_process_components.py:364-371); torch fp64 sum",
    "adamw_step": "torch.optim.AdamW on CPU: bitwise with torch's own sqrt injected, within "
    "1e-6 relative otherwise; closed form of step 1",
    "adamw_scalars": "with adamw_step: the step matches torch.optim.AdamW bitwise only when these host "
    "scalars are the ones torch forms (test_oracle_adamw.py), and step 1's closed form fixes them",
    "unpack_full": "round trip: the concatenated pack_shard pieces unpack to the original tensors bitwise "
    "for G = 1, 2, 3, 4 and 7 (test_host_logic.py)",
    "f32_to_bf16": "torch Tensor.to(torch.bfloat16) bitwise on specials and random values",
    "sgd_step": "torch.optim.SGD(foreach=False) on CPU, bitwise, with and without momentum, "
    "weight decay, dampening and Nesterov; closed form of a plain step",
    "read_range": "reference known answers: shards_overlapping [(0,(0,3)),(1,(3,1))] "
    "(test_checkpoint_format.py:242-247); bitwise re-slicing of the global flat vector",
    "local_share": "torch Tensor.to(reduce dtype) + div + add + padding zero in fp32, bf16 and fp16, "
    "bitwise (order-free for G <= 2; collectives.py:593-594); padding tail exactly 0.0 "
    "(test_fsdp.py:477-481); in float64 against torch's float64 ops bitwise and, for G a power of two, "
    "the exact rational mean rounded once to fp32",
    "no_sync_accumulate": "torch's own CPU sequence of fsdp.py:733-749 (to(reduce dtype), clone, add_, "
    "grad + accumulator) in fp32, bf16 and fp16, bitwise on signed zeros, subnormals, overflow and "
    "random values; in float64 bitwise against torch and equal to the exact sum",
    "round_to": "torch Tensor.to(bfloat16 / float16).to(float32) bitwise on specials and random values",
    "f16_nan_rules": "torch's vectorised CPU Tensor.to (x86 F16C) bitwise on all 65,536 fp16 bit patterns "
    "(widening) and on NaN payloads of both signs, signalling and quiet (narrowing)",
    "adamw_step_f64": "torch.optim.AdamW(foreach=False) stepping float64 CPU tensors: bitwise over 10 steps on "
    "both lerp branches, with and without weight decay and clip, with torch's own sqrt injected, within 1e-15 "
    "relative otherwise; step 1's closed form; a separately rounded addcmul product is shown to differ",
    "sgd_step_f64": "torch.optim.SGD(foreach=False) stepping float64 CPU tensors, bitwise, for every "
    "combination of momentum, dampening, weight decay and Nesterov",
    "sqnorm_f64": "math.fsum of the rounded double squares; torch's float64 pow(2).sum()",
    "clip_multiplier64": "the reference's Python-double coefficient: known answer norm 6 -> 1/(6+1e-6), "
    "and torch's grad.mul_(coef) on float64 tensors bitwise",
}


def library() -> ctypes.CDLL:
    """The C restatement, built on first use when missing."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(_LIB_PATH):
            subprocess.run(["make", "-C", _HERE], check=True, capture_output=True)
        lib = ctypes.CDLL(_LIB_PATH)
        vp, f32p, u16p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint16)
        i64, ci, cf = ctypes.c_int64, ctypes.c_int, ctypes.c_float
        lib.oracle_adamw.restype = None
        lib.oracle_adamw.argtypes = [vp, vp, vp, vp, i64, ci, ci] + [cf] * 9 + [f32p, vp]
        lib.oracle_sgd.restype = None
        lib.oracle_sgd.argtypes = [vp, vp, vp, i64, ci, ci, cf, cf, ci, cf, ci, cf, cf, ci, cf, vp, ci]
        lib.oracle_sqnorm.restype = ctypes.c_double
        lib.oracle_sqnorm.argtypes = [vp, i64, ci, cf]
        lib.oracle_round.restype = None
        lib.oracle_round.argtypes = [f32p, f32p, i64, ci]
        lib.oracle_f32_to_bf16.restype = None
        lib.oracle_f32_to_bf16.argtypes = [f32p, u16p, i64]
        lib.oracle_f32_to_f16.restype = None
        lib.oracle_f32_to_f16.argtypes = [f32p, u16p, i64]
        cd = ctypes.c_double
        lib.oracle_adamw_f64.restype = None
        lib.oracle_adamw_f64.argtypes = [vp, vp, vp, vp, i64, cd, cd, cd, cd, cd, cd, cd, cd, cd, vp, vp]
        lib.oracle_sgd_f64.restype = None
        lib.oracle_sgd_f64.argtypes = [vp, vp, vp, i64, cd, cd, ci, cd, ci, cd, cd, ci, cd, vp]
        lib.oracle_sqnorm_f64.restype = cd
        lib.oracle_sqnorm_f64.argtypes = [vp, i64]
        _LIB = lib
    return _LIB


def _f32(a: np.ndarray) -> ctypes.POINTER(ctypes.c_float):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u16(a: np.ndarray) -> ctypes.POINTER(ctypes.c_uint16):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def _vp(a: np.ndarray | None) -> ctypes.c_void_p | None:
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


#: Dtype names and the codes the C restatement (and libhbt.so) use for them.
DTYPE_CODES = {"float32": 0, "bfloat16": 1, "float16": 2}


def _storage(a: np.ndarray, dtype: str) -> None:
    """``a`` holds ``dtype`` values: float32 values, or 2-byte bit patterns as uint16."""
    expected = np.float32 if dtype == "float32" else np.uint16
    assert a.dtype == expected and a.flags.c_contiguous, (a.dtype, dtype)


def to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values rounded to ``dtype`` (nearest even), as that dtype's storage: float32
    values for ``"float32"``, uint16 bit patterns for ``"bfloat16"`` / ``"float16"``."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "float32":
        return x.copy()
    out = np.empty(x.shape, dtype=np.uint16)
    fn = library().oracle_f32_to_bf16 if dtype == "bfloat16" else library().oracle_f32_to_f16
    fn(_f32(x), _u16(out), x.size)
    return out


def from_bits(a: np.ndarray, dtype: str) -> np.ndarray:
    """The fp32 values of ``dtype`` storage (exact widening)."""
    if dtype == "float32":
        return np.asarray(a, dtype=np.float32)
    if dtype == "bfloat16":
        return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------------------
# AdamW
# ---------------------------------------------------------------------------------------
def adamw_scalars(
    *, lr: float, beta1: float, beta2: float, eps: float, weight_decay: float, step: float
) -> tuple[float, float, float, float, float, float, float]:
    """Host scalars of one AdamW step, formed in double as torch/optim/adam.py:416-547 does.

    Returns ``(decay, lerp_weight, beta2, one_minus_beta2, bias_correction2_sqrt, eps,
    neg_step_size)``; the kernels round each to fp32.
    """
    bias_correction1 = 1 - beta1**step
    bias_correction2 = 1 - beta2**step
    step_size = lr / bias_correction1
    decay = 1 - lr * weight_decay if weight_decay != 0 else 1.0
    return (decay, 1 - beta1, beta2, 1 - beta2, bias_correction2**0.5, eps, -step_size)


def _grad_dtype(g: np.ndarray, dtype: str, grad_dtype: str | None) -> str:
    if grad_dtype is not None:
        return grad_dtype
    if g.dtype == np.float32:
        return "float32"
    return "bfloat16" if dtype == "float32" else dtype


def adamw_step(
    p: np.ndarray,
    g: np.ndarray,
    m: np.ndarray,
    v: np.ndarray,
    scalars: Sequence[float],
    *,
    unscale: float = 1.0,
    grad_mul: float = 1.0,
    sqrt_override: np.ndarray | None = None,
    dtype: str = "float32",
    grad_dtype: str | None = None,
    grad_out: np.ndarray | None = None,
) -> None:
    """One AdamW step in place on ``p, m, v`` of ``dtype`` (float32 arrays, or uint16 bit
    patterns of bfloat16 / float16).  ``g`` is float32, or uint16 bits of ``grad_dtype``
    (bfloat16 by default for fp32 parameters, else the parameters' dtype).  The unscale
    and clip multiplies are rounded to the gradient's dtype; ``grad_out`` (the gradient's
    storage dtype) receives the scaled gradient."""
    gdt = _grad_dtype(g, dtype, grad_dtype)
    for a in (p, m, v):
        _storage(a, dtype)
    g = np.ascontiguousarray(g)
    _storage(g, gdt)
    if grad_out is not None:
        _storage(grad_out, gdt)
    override = None if sqrt_override is None else _f32(np.ascontiguousarray(sqrt_override, np.float32))
    library().oracle_adamw(_vp(p), _vp(g), _vp(m), _vp(v), p.size, DTYPE_CODES[dtype], DTYPE_CODES[gdt],
                           unscale, grad_mul, *scalars, override, _vp(grad_out))


def sgd_step(
    p: np.ndarray,
    g: np.ndarray,
    buf: np.ndarray | None,
    *,
    lr: float,
    momentum: float = 0.0,
    dampening: float = 0.0,
    weight_decay: float = 0.0,
    nesterov: bool = False,
    first: bool = False,
    unscale: float = 1.0,
    grad_mul: float = 1.0,
    dtype: str = "float32",
    grad_dtype: str | None = None,
    grad_out: np.ndarray | None = None,
    remainder: bool = False,
) -> None:
    """One SGD step in place on ``p`` (and ``buf``) of ``dtype``; torch's scalars rounded
    to fp32, and each alpha to ``dtype``.  Storage as for :func:`adamw_step`.
    ``remainder`` gives the arithmetic of torch's scalar remainder loop on 2-byte tensors
    (each alpha product rounded to ``dtype`` before the add) instead of its vectorised
    body's, which the kernels follow."""
    gdt = _grad_dtype(g, dtype, grad_dtype)
    _storage(p, dtype)
    g = np.ascontiguousarray(g)
    _storage(g, gdt)
    mode = 0 if momentum == 0 else (1 if first else 2)
    if mode:
        assert buf is not None
        _storage(buf, dtype)
    if grad_out is not None:
        _storage(grad_out, gdt)
    library().oracle_sgd(_vp(p), _vp(g), _vp(buf) if mode else None, p.size, DTYPE_CODES[dtype], DTYPE_CODES[gdt],
                         unscale, grad_mul, int(weight_decay != 0), weight_decay, mode, momentum, 1 - dampening,
                         int(nesterov), -lr, _vp(grad_out), int(remainder))


# ---------------------------------------------------------------------------------------
# norm and clip
# ---------------------------------------------------------------------------------------
def sqnorm(g: np.ndarray, *, unscale: float = 1.0, dtype: str | None = None) -> float:
    """Compensated fp64 sum of squares of ``R(g * unscale)``: ``g`` float32, or uint16 bits
    of ``dtype`` (bfloat16 by default), the product rounded to that dtype."""
    g = np.ascontiguousarray(g)
    gdt = "float32" if g.dtype == np.float32 else (dtype or "bfloat16")
    _storage(g, gdt)
    return float(library().oracle_sqnorm(_vp(g), g.size, DTYPE_CODES[gdt], unscale))


def clip_multiplier(norm: float, max_norm: float) -> float:
    """fp32 value the gradients are multiplied by (sharded_optimizer.py:331-337): the
    Python-double coefficient rounded to fp32 when it is below 1, else exactly 1."""
    if max_norm <= 0:
        return 1.0
    coef = float(max_norm) / (float(norm) + 1e-6)
    return float(np.float32(coef)) if coef < 1.0 else 1.0


def clip_multiplier64(norm: float, max_norm: float) -> float:
    """The double a float64 gradient is multiplied by (sharded_optimizer.py:331-337): the
    Python-double coefficient itself when it is below 1, else exactly 1."""
    if max_norm <= 0:
        return 1.0
    coef = float(max_norm) / (float(norm) + 1e-6)
    return coef if coef < 1.0 else 1.0


def _f64(a: np.ndarray) -> ctypes.c_void_p:
    assert a.dtype == np.float64 and a.flags.c_contiguous, a.dtype
    return ctypes.c_void_p(a.ctypes.data)


def adamw_step_f64(p, g, m, v, scalars, *, unscale=1.0, grad_mul=1.0, sqrt_override=None, grad_out=None) -> None:
    """One AdamW step in place on float64 ``p, m, v`` with float64 ``g`` and the double
    scalars of :func:`adamw_scalars`, as torch steps float64 tensors."""
    g = np.ascontiguousarray(g, np.float64)
    root = None if sqrt_override is None else np.ascontiguousarray(sqrt_override, np.float64)
    library().oracle_adamw_f64(_f64(p), _f64(g), _f64(m), _f64(v), p.size, unscale, grad_mul, *scalars,
                               None if root is None else _f64(root), None if grad_out is None else _f64(grad_out))


def sgd_step_f64(p, g, buf, *, lr, momentum=0.0, dampening=0.0, weight_decay=0.0, nesterov=False, first=False,
                 unscale=1.0, grad_mul=1.0, grad_out=None) -> None:
    """One SGD step in place on float64 ``p`` (and ``buf``), the alphas unrounded."""
    g = np.ascontiguousarray(g, np.float64)
    mode = 0 if momentum == 0 else (1 if first else 2)
    library().oracle_sgd_f64(_f64(p), _f64(g), _f64(buf) if mode else None, p.size, unscale, grad_mul,
                             int(weight_decay != 0), weight_decay, mode, momentum, 1 - dampening, int(nesterov),
                             -lr, None if grad_out is None else _f64(grad_out))


def sqnorm_f64(g: np.ndarray) -> float:
    """Compensated sum of the rounded double squares of float64 ``g``."""
    g = np.ascontiguousarray(g, np.float64)
    return float(library().oracle_sqnorm_f64(_f64(g), g.size))


def f16_nan_rules():
    """(widen, narrow): fp16 -> fp32 and fp32 -> fp16 on bit patterns, NaN bits included.

    Non-NaN values convert as IEEE does (numpy's exact widening, round-to-nearest-even
    narrowing with overflow to infinity).  A NaN keeps its sign and gets the quiet bit:
    widening keeps the 10-bit payload as the top of the 23-bit one, narrowing keeps the
    payload's top 10 bits.  These are the rules of x86 F16C, which torch's vectorised CPU
    conversions use (the reference's fp16 casts, ``parallel/fsdp.py:578-579``, ``:734-735``).
    """

    def widen(bits16: np.ndarray) -> np.ndarray:
        b = np.asarray(bits16, np.uint16)
        with np.errstate(invalid="ignore"):
            out = b.view(np.float16).astype(np.float32).view(np.uint32).copy()
        b32 = b.astype(np.uint32)
        nan = ((b32 & 0x7C00) == 0x7C00) & ((b32 & 0x03FF) != 0)
        out[nan] = ((b32[nan] & 0x8000) << 16) | 0x7FC00000 | ((b32[nan] & 0x03FF) << 13)
        return out

    def narrow(bits32: np.ndarray) -> np.ndarray:
        u = np.asarray(bits32, np.uint32)
        with np.errstate(over="ignore", invalid="ignore"):
            out = u.view(np.float32).astype(np.float16).view(np.uint16).copy()
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        out[nan] = (((u[nan] >> 16) & 0x8000) | 0x7E00 | ((u[nan] >> 13) & 0x03FF)).astype(np.uint16)
        return out

    return widen, narrow


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) of ``x`` rounded to nearest even, NaN -> 0x7FC0."""
    return to_bits(x, "bfloat16")


# ---------------------------------------------------------------------------------------
# layout, pack, unpack
# ---------------------------------------------------------------------------------------
def flat_layout(numels: Sequence[int]) -> tuple[list[int], int]:
    """Offsets (exclusive prefix sum) and total of a flat buffer (utils/tensors.py:137-196)."""
    sizes = np.asarray(list(numels), dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]]) if sizes.size else np.zeros(0, np.int64)
    return [int(o) for o in offsets], int(sizes.sum())


def even_shards(total: int, group: int) -> tuple[int, int, int]:
    """``(shard_numel, padded_numel, padding)`` (parallel/fsdp.py:395-399)."""
    shard = (total + group - 1) // group
    return shard, shard * group, shard * group - total


def pack_shard(tensors: Sequence[np.ndarray], group: int, rank: int) -> np.ndarray:
    """Rank ``rank``'s slice of the zero-padded concatenation (parallel/fsdp.py:434-454)."""
    flat = np.concatenate([np.ascontiguousarray(t).reshape(-1) for t in tensors])
    shard, padded, _ = even_shards(flat.size, group)
    full = np.zeros(padded, dtype=flat.dtype)
    full[: flat.size] = flat
    return full[rank * shard : (rank + 1) * shard].copy()


def unpack_full(flat: np.ndarray, shapes: Sequence[tuple[int, ...]]) -> list[np.ndarray]:
    """Per-tensor copies of a flat buffer (parallel/fsdp.py:912-925)."""
    out, cursor = [], 0
    for shape in shapes:
        n = int(np.prod(shape)) if len(shape) else 1
        out.append(flat[cursor : cursor + n].reshape(shape).copy())
        cursor += n
    return out


def bucket_layout(
    named: Sequence[tuple[str, int, int]], cap_bytes: int
) -> list[list[tuple[str, int, int]]]:
    """Greedy buckets over ``(name, numel, element_size)`` in REVERSE order
    (parallel/ddp.py:397-463): close a bucket before a parameter that would push it
    past ``cap_bytes``; returns ``[(name, offset, numel), ...]`` per bucket."""
    buckets: list[list[tuple[str, int, int]]] = []
    current: list[tuple[str, int, int]] = []
    used = 0
    for name, numel, esize in reversed(list(named)):
        nbytes = numel * esize
        if current and used + nbytes > cap_bytes:
            buckets.append(current)
            current, used = [], 0
        offset = sum(n for _, _, n in current)
        current.append((name, offset, numel))
        used += nbytes
    if current:
        buckets.append(current)
    return buckets


def round_to(x: np.ndarray, reduce: str = "float32") -> np.ndarray:
    """fp32 ``x`` rounded to the dtype ``reduce`` names (round to nearest even) and widened
    back, exactly: the value a torch op whose result has that dtype holds."""
    x = np.asarray(x, dtype=np.float32)
    if reduce == "float32":
        return x
    if reduce in ("bfloat16", "float16"):
        flat = np.ascontiguousarray(x).reshape(-1)
        out = np.empty_like(flat)
        library().oracle_round(_f32(flat), _f32(out), flat.size, DTYPE_CODES[reduce])
        return out.reshape(x.shape)
    raise ValueError(f"unknown reduce dtype {reduce!r}")


def local_share(rank_grads: Sequence[np.ndarray], rank: int, shard: int, valid: int,
                divisor: float, reduce: str = "float32", out: str = "float32") -> np.ndarray:
    """fp32 shard ``rank`` of the AVG reduce-scatter in the reduce dtype, summed in rank
    order (parallel/fsdp.py:733-769, distributed/collectives.py:593-594): each rank's
    slice cast to ``reduce``, divided by ``divisor`` and added, every result rounded to
    ``reduce``; then widened to fp32 with the padding tail zeroed.  ``rank_grads`` hold
    each rank's padded full gradient widened to fp32 (bf16 and fp16 widen exactly).

    ``reduce="float64"`` widens each slice to float64 (the rank grads may then also be
    float64 arrays, the no_sync accumulator's rows), divides and sums in float64 and
    rounds the sum once to fp32 (``Tensor.to``, round to nearest even), or, with
    ``out="float64"`` (a float64 master), keeps the float64 sum."""
    if reduce == "float64":
        div64 = np.float64(divisor)
        with np.errstate(over="ignore", invalid="ignore"):
            acc64 = np.asarray(rank_grads[0], dtype=np.float64)[rank * shard : (rank + 1) * shard] / div64
            for g in rank_grads[1:]:
                acc64 = acc64 + np.asarray(g, dtype=np.float64)[rank * shard : (rank + 1) * shard] / div64
            result = acc64.copy() if out == "float64" else acc64.astype(np.float32)
        result[valid:] = 0.0
        return result
    div = np.float32(divisor)

    def term(g: np.ndarray) -> np.ndarray:
        x = round_to(np.asarray(g, dtype=np.float32)[rank * shard : (rank + 1) * shard], reduce)
        return round_to(x / div, reduce)

    with np.errstate(over="ignore", invalid="ignore"):
        acc = term(rank_grads[0])
        for g in rank_grads[1:]:
            acc = round_to(acc + term(g), reduce)
    acc = np.array(acc, dtype=np.float32)
    acc[valid:] = 0.0
    return acc


def no_sync_accumulate(micro_grads: Sequence[np.ndarray], reduce: str = "float32") -> np.ndarray:
    """The gradient one rank reduces after ``no_sync`` accumulation in the reduce dtype
    (parallel/fsdp.py:733-749), as fp32 values exactly representable in ``reduce``.
    ``micro_grads`` are the micro-batches' gradients in order, widened to fp32 (bf16 and
    fp16 widen exactly); all but the last ran inside ``no_sync``.  Each is cast to
    ``reduce``; the first is kept as it is (``clone``), each later one inside ``no_sync``
    is added to it (``add_``), and the last, synchronising one is added in front
    (``grad + accumulator``), every sum rounded to ``reduce``.  For ``reduce="float64"``
    the sums run in float64 and the float64 array is returned."""
    if reduce == "float64":
        acc64 = np.array(micro_grads[0], dtype=np.float64, copy=True)
        with np.errstate(over="ignore", invalid="ignore"):
            for g in micro_grads[1:-1]:
                acc64 = acc64 + np.asarray(g, dtype=np.float64)
            if len(micro_grads) > 1:
                acc64 = np.asarray(micro_grads[-1], dtype=np.float64) + acc64
        return acc64
    acc = np.array(round_to(micro_grads[0], reduce), dtype=np.float32, copy=True)
    if len(micro_grads) == 1:
        return acc
    with np.errstate(over="ignore", invalid="ignore"):  # IEEE overflow to +-inf is the answer
        for g in micro_grads[1:-1]:
            acc = round_to(np.add(acc, round_to(g, reduce), dtype=np.float32), reduce)
        return round_to(np.add(round_to(micro_grads[-1], reduce), acc, dtype=np.float32), reduce)


def read_range(shards: Sequence[tuple[int, np.ndarray]], start: int, length: int) -> np.ndarray:
    """Elements ``[start, start+length)`` of a tensor stored as ``(offset, data)`` pieces
    (checkpoint/reshard.py:200-305): intersect each piece, copy in offset order."""
    out = None
    cursor = start
    for offset, data in sorted(shards, key=lambda s: s[0]):
        lo, hi = max(offset, start), min(offset + data.size, start + length)
        if hi <= lo:
            continue
        if lo != cursor:
            raise ValueError(f"gap at {cursor}")
        if out is None:
            out = np.empty(length, dtype=data.dtype)
        out[lo - start : hi - start] = data[lo - offset : hi - offset]
        cursor = hi
    if cursor != start + length:
        raise ValueError("range not covered")
    return out if out is not None else np.empty(0)
