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
    "PINNED_BY",
    "adamw_scalars",
    "adamw_step",
    "bucket_layout",
    "clip_multiplier",
    "even_shards",
    "f32_to_bf16",
    "flat_layout",
    "library",
    "local_share",
    "no_sync_accumulate",
    "pack_shard",
    "read_range",
    "round_to",
    "sgd_step",
    "sqnorm",
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
}


def library() -> ctypes.CDLL:
    """The C restatement, built on first use when missing."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(_LIB_PATH):
            subprocess.run(["make", "-C", _HERE], check=True, capture_output=True)
        lib = ctypes.CDLL(_LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        lib.oracle_adamw_f32.restype = None
        lib.oracle_adamw_f32.argtypes = [f32p, f32p, f32p, f32p, ctypes.c_int64] + [
            ctypes.c_float
        ] * 9 + [f32p]
        lib.oracle_adamw_bf16grad.restype = None
        lib.oracle_adamw_bf16grad.argtypes = [f32p, u16p, f32p, f32p, ctypes.c_int64] + [
            ctypes.c_float
        ] * 9
        lib.oracle_sgd.restype = None
        lib.oracle_sgd.argtypes = [f32p, f32p, f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_float,
                                   ctypes.c_float, ctypes.c_int, ctypes.c_float]
        lib.oracle_sqnorm_f32.restype = ctypes.c_double
        lib.oracle_sqnorm_f32.argtypes = [f32p, ctypes.c_int64, ctypes.c_float]
        lib.oracle_sqnorm_bf16.restype = ctypes.c_double
        lib.oracle_sqnorm_bf16.argtypes = [u16p, ctypes.c_int64, ctypes.c_float]
        lib.oracle_f32_to_bf16.restype = None
        lib.oracle_f32_to_bf16.argtypes = [f32p, u16p, ctypes.c_int64]
        _LIB = lib
    return _LIB


def _f32(a: np.ndarray) -> ctypes.POINTER(ctypes.c_float):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u16(a: np.ndarray) -> ctypes.POINTER(ctypes.c_uint16):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


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
) -> None:
    """One AdamW step in place on fp32 ``p, m, v`` (``g`` fp32, or bf16 bits as uint16)."""
    for a in (p, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    n = p.size
    lib = library()
    if g.dtype == np.uint16:
        assert sqrt_override is None
        lib.oracle_adamw_bf16grad(_f32(p), _u16(g), _f32(m), _f32(v), n, unscale, grad_mul, *scalars)
        return
    assert g.dtype == np.float32
    override = None if sqrt_override is None else _f32(np.ascontiguousarray(sqrt_override, np.float32))
    lib.oracle_adamw_f32(_f32(p), _f32(np.ascontiguousarray(g)), _f32(m), _f32(v), n, unscale, grad_mul,
                         *scalars, override)


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
) -> None:
    """One SGD step in place on fp32 ``p`` (and ``buf``), torch's scalars rounded to fp32."""
    assert p.dtype == np.float32 and p.flags.c_contiguous and g.dtype == np.float32
    mode = 0 if momentum == 0 else (1 if first else 2)
    if mode:
        assert buf is not None and buf.dtype == np.float32 and buf.flags.c_contiguous
    b = _f32(buf) if buf is not None else None
    library().oracle_sgd(_f32(p), _f32(np.ascontiguousarray(g)), b, p.size, unscale, grad_mul,
                         int(weight_decay != 0), weight_decay, mode, momentum, 1 - dampening,
                         int(nesterov), -lr)


# ---------------------------------------------------------------------------------------
# norm and clip
# ---------------------------------------------------------------------------------------
def sqnorm(g: np.ndarray, *, unscale: float = 1.0) -> float:
    """Compensated fp64 sum of squares of ``g * unscale`` (fp32, or bf16 bits as uint16)."""
    g = np.ascontiguousarray(g)
    if g.dtype == np.uint16:
        return float(library().oracle_sqnorm_bf16(_u16(g), g.size, unscale))
    assert g.dtype == np.float32
    return float(library().oracle_sqnorm_f32(_f32(g), g.size, unscale))


def clip_multiplier(norm: float, max_norm: float) -> float:
    """fp32 value the gradients are multiplied by (sharded_optimizer.py:331-337): the
    Python-double coefficient rounded to fp32 when it is below 1, else exactly 1."""
    if max_norm <= 0:
        return 1.0
    coef = float(max_norm) / (float(norm) + 1e-6)
    return float(np.float32(coef)) if coef < 1.0 else 1.0


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) of ``x`` rounded to nearest even, NaN -> 0x7FC0."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    library().oracle_f32_to_bf16(_f32(x), _u16(out), x.size)
    return out


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
    if reduce == "bfloat16":
        return (f32_to_bf16(x).astype(np.uint32) << 16).view(np.float32)
    if reduce == "float16":
        with np.errstate(over="ignore"):
            return x.astype(np.float16).astype(np.float32)
    raise ValueError(f"unknown reduce dtype {reduce!r}")


def local_share(rank_grads: Sequence[np.ndarray], rank: int, shard: int, valid: int,
                divisor: float, reduce: str = "float32") -> np.ndarray:
    """fp32 shard ``rank`` of the AVG reduce-scatter in the reduce dtype, summed in rank
    order (parallel/fsdp.py:733-769, distributed/collectives.py:593-594): each rank's
    slice cast to ``reduce``, divided by ``divisor`` and added, every result rounded to
    ``reduce``; then widened to fp32 with the padding tail zeroed.  ``rank_grads`` hold
    each rank's padded full gradient widened to fp32 (bf16 and fp16 widen exactly).

    ``reduce="float64"`` widens each slice to float64 (the rank grads may then also be
    float64 arrays, the no_sync accumulator's rows), divides and sums in float64 and
    rounds the sum once to fp32 (``Tensor.to``, round to nearest even)."""
    if reduce == "float64":
        div64 = np.float64(divisor)
        with np.errstate(over="ignore", invalid="ignore"):
            acc64 = np.asarray(rank_grads[0], dtype=np.float64)[rank * shard : (rank + 1) * shard] / div64
            for g in rank_grads[1:]:
                acc64 = acc64 + np.asarray(g, dtype=np.float64)[rank * shard : (rank + 1) * shard] / div64
            out = acc64.astype(np.float32)
        out[valid:] = 0.0
        return out
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
