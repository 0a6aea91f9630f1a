"""GPU parity of the element-wise entry points at sizes that exercise every tile path.

* ``hbt_grad_local_share`` and ``hbt_grad_local_share_sqnorm`` (the FSDP gradient
  local share, ``parallel/fsdp.py:704-781``, the latter with the norm partials of its
  output): bitwise against the oracle for G in {1, 3, 8}, fp32, bf16 and fp16 inputs,
  shards with full vector tiles, a partial tile at the valid/padding boundary, whole
  tiles of padding, and misaligned input and output addresses (scalar path); the
  partials sum to the oracle's squared norm within 1e-12.
* ``hbt_scale_inplace`` (the ``grad.mul_`` loops of ``optim/grad_scaler.py:181-186``
  and ``optim/sharded_optimizer.py:333-337``): bitwise against torch's own CPU
  ``mul_`` by a Python float, twice, in the tensor's dtype, over several tensors per
  launch, tails of every length and a misaligned view.
* ``hbt_scale_inplace_sqnorm`` (the loss scaler's unscale fused with its overflow
  check, ``optim/grad_scaler.py:181-200``): bitwise the two calls it replaces,
  ``hbt_scale_inplace`` then ``hbt_grad_sqnorm_partials``, in fp32, bf16 and fp16, over
  tails, multi-chunk tensors, misaligned views and IEEE specials, partials included.
* ``hbt_grad_local_share_accumulated`` (the reduction that ends a ``no_sync``
  accumulation, ``parallel/fsdp.py:747-769``): bitwise ``hbt_grad_accumulate`` over the
  rows followed by ``hbt_grad_local_share_sqnorm`` at rank offset 0, outputs and norm
  partials, for G in {1, 2, 3, 8}, every input / reduce / master dtype, padding, and a
  misaligned row (scalar path); an fp64 reduce dtype is refused.
* ``hbt_grad_accumulate`` (the ``no_sync`` accumulation of ``parallel/fsdp.py:738-749``):
  bitwise against torch's CPU ``add_`` (or the cast alone, for the first micro-batch)
  in an fp32, bf16 or fp16 accumulator, fp32, bf16 and fp16 gradients, tails of every
  length, a misaligned pair and IEEE specials.
The local share runs in each reduce dtype (fp32, bf16, fp16) against the oracle's.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import _native

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    return t.view({2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]).numpy().copy()


_REDUCE = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16",
           torch.float64: "float64"}


def _master_bits(t: torch.Tensor) -> np.ndarray:
    """Raw bits of a float32 (int32 view) or 2-byte (uint16 view) tensor."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("group", [1, 3, 8])
@pytest.mark.parametrize("misaligned", [False, True])
@pytest.mark.parametrize("reduce", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("master", [torch.float32, torch.bfloat16, torch.float16])
def test_local_share_tiles(device, in_dtype, group, misaligned, reduce, master):
    """The shard in every (input, reduce, master) dtype combination: the oracle's
    reduce-dtype sum, cast to the master dtype as Tensor.to casts (``fsdp.py:763-764``)."""
    if master != torch.float32 and (group == 3 or reduce == torch.float16 and in_dtype == torch.bfloat16):
        pytest.skip("2-byte masters: a representative subset of the combinations")
    lib = _native.library()
    shard = 20_000
    gen = torch.Generator(device=device).manual_seed(group)
    lead = 1 if misaligned else 0
    # Each rank's padded full gradient (group * shard elements), optionally one element
    # into its allocation so the vector path is not taken.
    storage = [(torch.randn(group * shard + lead, device=device, generator=gen) * 1e-2).to(in_dtype)
               for _ in range(group)]
    grads = [s[lead:] for s in storage]
    host = [g.float().cpu().numpy() for g in grads]
    out_storage = torch.full((shard + lead,), 7.0, device=device, dtype=master)
    out = out_storage[lead:]
    divisor = float(group) if group > 1 else 1.0
    master_name = _REDUCE[master]
    for rank in sorted({0, group - 1}):
        for valid in (shard, shard - 1537, 700, 0):
            status = lib.hbt_grad_local_share(
                _native.pointer_array([g.data_ptr() for g in grads]), group, rank, shard, valid,
                _native.dtype_code(in_dtype), _native.dtype_code(reduce), divisor, _native.dtype_code(master),
                ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(_native.stream_of(device)),
            )
            _native.check(status, "test.local_share")
            expect32 = oracle.local_share(host, rank, shard, valid, divisor, _REDUCE[reduce])
            expect = oracle.to_bits(expect32, master_name)
            expect = expect.view(np.int32) if master == torch.float32 else expect
            assert np.array_equal(_master_bits(out), expect), (rank, valid)
            # the fused entry point: the same shard, plus its squared-norm partials
            chunk = 32768 if master == torch.float32 else 65536
            partials = torch.full((-(-valid // chunk) + -(-(shard - valid) // chunk) or 1,), 7.0,
                                  dtype=torch.float64, device=device)
            tile_sums = torch.empty(-(-shard // 256), dtype=torch.float64, device=device)
            out.fill_(7.0)
            status = lib.hbt_grad_local_share_sqnorm(
                _native.pointer_array([g.data_ptr() for g in grads]), group, rank, shard, valid,
                _native.dtype_code(in_dtype), _native.dtype_code(reduce), divisor, _native.dtype_code(master),
                ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(partials.data_ptr()),
                ctypes.c_void_p(tile_sums.data_ptr()), ctypes.c_void_p(_native.stream_of(device)),
            )
            _native.check(status, "test.local_share_sqnorm")
            assert np.array_equal(_master_bits(out), expect), (rank, valid)
            ref = oracle.sqnorm(oracle.from_bits(oracle.to_bits(expect32, master_name), master_name))
            got = float(partials.sum())
            assert abs(got - ref) <= 1e-12 * max(ref, 1e-300), (rank, valid, got, ref)
    assert float(out_storage[:lead].float().sum()) == 7.0 * lead  # nothing written before the output


@pytest.mark.parametrize("master", [torch.float32, torch.bfloat16])
def test_local_share_partials_chunk_by_chunk(device, master):
    """Each norm partial of ``hbt_grad_local_share_sqnorm`` is the squared norm of its own
    chunk of the output: chunks of 32,768 fp32 (65,536 2-byte) elements from 0 up to
    ``valid``, then zero partials over the padding.  The shard spans many chunks and 1,172
    tiles, so a tile sum counted in the wrong chunk (the sums are stored in a permuted
    order and read back through it) changes individual partials, which a check of their
    total would not see.  Each partial is within 1e-12 of a brute-force fp64 sum."""
    import math

    lib = _native.library()
    group, shard, valid = 4, 300_000, 250_001
    gen = torch.Generator(device=device).manual_seed(17)
    grads = [(torch.randn(group * shard, device=device, generator=gen) * 1e-2).to(torch.bfloat16)
             for _ in range(group)]
    host = [g.float().cpu().numpy() for g in grads]
    out = torch.empty(shard, device=device, dtype=master)
    chunk = 32768 if master == torch.float32 else 65536
    valid_chunks, pad_chunks = -(-valid // chunk), -(-(shard - valid) // chunk)
    partials = torch.full((valid_chunks + pad_chunks,), 7.0, dtype=torch.float64, device=device)
    tile_sums = torch.empty(-(-shard // 256), dtype=torch.float64, device=device)
    for rank in (0, group - 1):
        status = lib.hbt_grad_local_share_sqnorm(
            _native.pointer_array([g.data_ptr() for g in grads]), group, rank, shard, valid,
            _native.dtype_code(torch.bfloat16), _native.dtype_code(torch.float32), float(group),
            _native.dtype_code(master), ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(partials.data_ptr()),
            ctypes.c_void_p(tile_sums.data_ptr()), ctypes.c_void_p(_native.stream_of(device)),
        )
        _native.check(status, "test.local_share_sqnorm")
        values = out.double().cpu().numpy()
        got = partials.cpu().numpy()
        for c in range(valid_chunks):
            ref = math.fsum(float(x) * float(x) for x in values[c * chunk : min((c + 1) * chunk, valid)])
            assert abs(got[c] - ref) <= 1e-12 * ref, (rank, c, got[c], ref)
        assert np.all(got[valid_chunks:] == 0.0) and np.all(values[valid:] == 0.0), rank
        expect = oracle.local_share(host, rank, shard, valid, float(group))
        assert np.array_equal(values.astype(np.float32), oracle.from_bits(oracle.to_bits(expect, _REDUCE[master]),
                                                                         _REDUCE[master])), rank


def _scale_reference(t: torch.Tensor, unscale: float, mul: float) -> torch.Tensor:
    """The reference's two in-place multiplies by Python floats, on the CPU in t's dtype."""
    return t.detach().cpu().clone().mul_(unscale).mul_(mul)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("factors", [(1.0 / 65536.0, 0.31622776601683794), (1.0, 0.31622776601683794), (0.5, 1.0)])
def test_scale_inplace_tiles(device, dtype, factors):
    lib = _native.library()
    gen = torch.Generator(device=device).manual_seed(3)
    sizes = [1, 7, 511, 512, 513, 4097, 100_003]
    base = torch.randn(sum(sizes) + 1, device=device, generator=gen).mul_(65536.0 * 1e-3).to(dtype)
    base[5] = float("inf")
    base[600] = float("nan")
    base[700] = 1e-41  # fp32 denormal / bf16 underflow after scaling
    tensors, cursor = [], 1  # the first tensor starts one element in: misaligned
    for n in sizes:
        tensors.append(base[cursor : cursor + n])
        cursor += n
    before = [t.detach().cpu().clone() for t in tensors]
    lead = _bits(base[:1])
    unscale, mul = factors  # the loss scaler's unscale and the clip; one of them alone
    grad_mul = torch.tensor([mul], dtype=torch.float32, device=device)
    status = lib.hbt_scale_inplace(
        _native.pointer_array([t.data_ptr() for t in tensors]), _native.int64_array(sizes), len(sizes),
        _native.dtype_code(dtype), unscale, ctypes.c_void_p(grad_mul.data_ptr()),
        ctypes.c_void_p(_native.stream_of(device)),
    )
    _native.check(status, "test.scale_inplace")
    # torch multiplies by the fp32 rounding of the Python float in fp32 arithmetic
    mul32 = float(np.float32(mul))
    for t, b in zip(tensors, before):
        expect = _scale_reference(b, unscale, mul32)
        got = t.detach().cpu()
        nan = torch.isnan(expect)
        assert torch.equal(torch.isnan(got), nan)
        assert np.array_equal(_bits(got)[~nan.numpy()], _bits(expect)[~nan.numpy()])
    assert np.array_equal(_bits(base[:1]), lead)  # the element before the first tensor is untouched


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("specials", [False, True])
def test_scale_inplace_sqnorm_is_the_two_calls(device, dtype, specials):
    lib = _native.library()
    gen = torch.Generator(device=device).manual_seed(9)
    sizes = [1, 7, 4097, 65536, 3 * 65536 + 5, 300_001]
    base = (torch.randn(sum(sizes) + 2, device=device, generator=gen) * 300.0).to(dtype)
    if specials:
        base[9] = float("inf")
        base[5000] = float("nan")
        base[70_000] = -float("inf")
    tensors_a, tensors_b, cursor = [], [], 1  # the first tensor starts one element in: misaligned
    twin = base.clone()
    for n in sizes:
        tensors_a.append(base[cursor : cursor + n])
        tensors_b.append(twin[cursor : cursor + n])
        cursor += n
    code = _native.dtype_code(dtype)
    unscale = float(np.float32(1.0 / 1000.0))
    count = int(lib.hbt_norm_partials_count(_native.int64_array(sizes), len(sizes), code))
    stream = ctypes.c_void_p(_native.stream_of(device))
    # the two calls: the in-place unscale, then the norm partials of the result
    _native.check(lib.hbt_scale_inplace(_native.pointer_array([t.data_ptr() for t in tensors_a]),
                                        _native.int64_array(sizes), len(sizes), code, unscale, None, stream),
                  "test.scale_inplace")
    expect = torch.empty(count, dtype=torch.float64, device=device)
    _native.check(lib.hbt_grad_sqnorm_partials(_native.pointer_array([t.data_ptr() for t in tensors_a]),
                                               _native.int64_array(sizes), _native.double_array([1.0] * len(sizes)),
                                               len(sizes), code, 1.0, ctypes.c_void_p(expect.data_ptr()), stream),
                  "test.sqnorm")
    # the fused call
    got = torch.empty(count, dtype=torch.float64, device=device)
    scratch = torch.empty(max(1, count) * _native.PIECES_PER_NORM_CHUNK, dtype=torch.float64, device=device)
    _native.check(lib.hbt_scale_inplace_sqnorm(_native.pointer_array([t.data_ptr() for t in tensors_b]),
                                               _native.int64_array(sizes), len(sizes), code, unscale,
                                               ctypes.c_void_p(got.data_ptr()), ctypes.c_void_p(scratch.data_ptr()),
                                               stream),
                  "test.scale_inplace_sqnorm")
    torch.cuda.synchronize(device)
    assert np.array_equal(_bits(base), _bits(twin))  # every element, the untouched first one included
    assert np.array_equal(expect.cpu().numpy().view(np.int64), got.cpu().numpy().view(np.int64))
    assert bool(torch.isfinite(got).all()) != specials


@pytest.mark.parametrize("group", [1, 2, 3, 8])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("reduce", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("master", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("misaligned", [False, True])
def test_local_share_accumulated_is_accumulate_then_share(device, group, in_dtype, reduce, master, misaligned):
    lib = _native.library()
    gen = torch.Generator(device=device).manual_seed(group * 7 + int(misaligned))
    shard = 3 * 65536 + 300 if not misaligned else 70_001
    valid = shard - 77
    rank = group - 1
    grads = [(torch.randn(group * shard, device=device, generator=gen) * 0.3).to(in_dtype) for _ in range(group)]
    stride = -(-shard // 64) * 64 + (1 if misaligned else 0)
    base = (torch.randn(group * stride, device=device, generator=gen) * 0.7).to(reduce)
    # IEEE specials in rank 0's slice and row: inf + -inf (a NaN), -0.0 + -0.0, a sum past the
    # reduce dtype's range, and an inf that stays one
    lo = rank * shard
    big = 6.0e4 if reduce == torch.float16 or in_dtype == torch.float16 else 3.0e38
    for e, gval, aval in ((5, float("inf"), -float("inf")), (6, -0.0, -0.0), (7, big, big), (8, float("inf"), 1.0)):
        grads[0][lo + e] = gval
        base[e] = aval
    rows_a = base.clone().view(group, stride)[:, :shard]
    rows_b = base.clone().view(group, stride)[:, :shard]
    code_in, code_red, code_out = (_native.dtype_code(d) for d in (in_dtype, reduce, master))
    stream = ctypes.c_void_p(_native.stream_of(device))
    divisor = float(group)
    chunk = 32768 if master == torch.float32 else 65536
    count = -(-valid // chunk) + -(-(shard - valid) // chunk)
    tiles = -(-shard // 256)

    def buffers():
        return (torch.empty(shard, dtype=master, device=device), torch.empty(max(1, count), dtype=torch.float64,
                device=device), torch.empty(tiles, dtype=torch.float64, device=device))

    # the two calls: the last micro-batch added into the rows, then the rows reduced
    offset = rank * shard * grads[0].element_size()
    _native.check(lib.hbt_grad_accumulate(_native.pointer_array([rows_a[q].data_ptr() for q in range(group)]),
                                          _native.pointer_array([g.data_ptr() + offset for g in grads]),
                                          _native.int64_array([shard] * group), group, code_red, code_in, 0, stream),
                  "test.accumulate")
    out_a, part_a, scratch_a = buffers()
    _native.check(lib.hbt_grad_local_share_sqnorm(_native.pointer_array([rows_a[q].data_ptr() for q in range(group)]),
                                                  group, 0, shard, valid, code_red, code_red, divisor, code_out,
                                                  out_a.data_ptr(), part_a.data_ptr(), scratch_a.data_ptr(), stream),
                  "test.share")
    # the fused call
    out_b, part_b, scratch_b = buffers()
    _native.check(lib.hbt_grad_local_share_accumulated(_native.pointer_array([g.data_ptr() for g in grads]),
                                                       _native.pointer_array([rows_b[q].data_ptr() for q in range(group)]),
                                                       group, rank, shard, valid, code_in, code_red, divisor, code_out,
                                                       out_b.data_ptr(), part_b.data_ptr(), scratch_b.data_ptr(), stream),
                  "test.share_accumulated")
    torch.cuda.synchronize(device)
    assert np.array_equal(_bits(out_a), _bits(out_b))  # NaNs included
    assert np.array_equal(part_a.cpu().numpy().view(np.int64), part_b.cpu().numpy().view(np.int64))
    assert bool(torch.isnan(out_b[5])) and float(out_b[valid:].abs().sum()) == 0.0
    if not misaligned and group == 2 and in_dtype == torch.float32:
        f64 = lib.hbt_grad_local_share_accumulated(_native.pointer_array([g.data_ptr() for g in grads]),
                                                   _native.pointer_array([rows_b[q].data_ptr() for q in range(group)]),
                                                   group, rank, shard, valid, code_in, 3, divisor, code_out,
                                                   out_b.data_ptr(), None, None, stream)
        assert f64 == -2 and b"F64" in lib.hbt_last_error()  # HBT_ERR_UNSUPPORTED


_SMALL_DTYPES = [(torch.float32, torch.float32, torch.float32), (torch.bfloat16, torch.float32, torch.float32),
                 (torch.bfloat16, torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16, torch.float32),
                 (torch.float32, torch.float32, torch.bfloat16)]


@pytest.mark.parametrize("tiles", [1, 2, 5, 16, 17])
@pytest.mark.parametrize("group", [1, 2, 3, 8])
@pytest.mark.parametrize("dtypes", _SMALL_DTYPES, ids=lambda d: "-".join(str(x).split(".")[1] for x in d))
@pytest.mark.parametrize("pad", [0, 3, 300])
def test_small_shard_local_share_is_the_two_launch_form(device, tiles, group, dtypes, pad):
    """A shard of at most 16 tiles of 256 elements takes one launch for its share and norm
    partials (one wave per tile in one workgroup); the shards here straddle that size, and
    300 padding elements make a one-tile shard all padding.  Outputs and partials must be
    bitwise those of the two-launch form (tiles, then their sums into partials), here
    ``hbt_grad_local_share_accumulated`` over all-zero rows, which always takes it (0 + x
    is x for these finite inputs, none of them -0.0): on aligned inputs (vector path) with
    finite values, and one element into the allocations (scalar path) with an inf planted.
    The output also matches the oracle, and the partials sum to its squared norm."""
    in_dtype, reduce, master = dtypes
    lib = _native.library()
    shard = tiles * 256 - 37
    valid = max(0, shard - pad)
    rank = group - 1
    code_in, code_red, code_out = (_native.dtype_code(d) for d in (in_dtype, reduce, master))
    stream = ctypes.c_void_p(_native.stream_of(device))
    chunk = 32768 if master == torch.float32 else 65536
    count = -(-valid // chunk) + -(-(shard - valid) // chunk)
    stride = -(-shard // 64) * 64
    rows = torch.zeros(group, stride, dtype=reduce, device=device)[:, :shard]
    for lead in (0, 1):
        gen = torch.Generator(device=device).manual_seed(tiles * 31 + group + lead)
        storage = [(torch.randn(group * shard + lead, device=device, generator=gen) * 0.3).to(in_dtype)
                   for _ in range(group)]
        grads = [t[lead:] for t in storage]
        if lead and valid > 1:
            grads[0][rank * shard + 1] = float("inf")

        def buffers():
            return (torch.full((shard,), 7.0, dtype=master, device=device),
                    torch.full((max(1, count),), 5.0, dtype=torch.float64, device=device),
                    torch.empty(tiles, dtype=torch.float64, device=device))

        out_a, part_a, scratch_a = buffers()
        _native.check(lib.hbt_grad_local_share_sqnorm(_native.pointer_array([g.data_ptr() for g in grads]), group,
                                                      rank, shard, valid, code_in, code_red, float(group), code_out,
                                                      out_a.data_ptr(), part_a.data_ptr(), scratch_a.data_ptr(),
                                                      stream),
                      "test.share_sqnorm")
        out_b, part_b, scratch_b = buffers()
        _native.check(lib.hbt_grad_local_share_accumulated(
            _native.pointer_array([g.data_ptr() for g in grads]),
            _native.pointer_array([rows[q].data_ptr() for q in range(group)]), group, rank, shard, valid, code_in,
            code_red, float(group), code_out, out_b.data_ptr(), part_b.data_ptr(), scratch_b.data_ptr(), stream),
            "test.share_accumulated")
        torch.cuda.synchronize(device)
        case = (tiles, group, pad, lead)
        assert np.array_equal(_bits(out_a), _bits(out_b)), case
        assert np.array_equal(part_a[:count].cpu().numpy().view(np.int64),
                              part_b[:count].cpu().numpy().view(np.int64)), case
        assert float(out_a[valid:].abs().sum()) == 0.0, case
        if reduce == torch.float32 and master == torch.float32:
            host = [g.float().cpu().numpy() for g in grads]
            expect = oracle.local_share(host, rank, shard, valid, float(group))
            assert np.array_equal(_bits(out_a), expect.view(np.int32)), case
        if valid and lead and valid > 1:
            assert math.isinf(float(part_a[0])), case
        elif valid:
            ref = float((out_a[:valid].double() ** 2).sum())
            assert abs(float(part_a[0]) - ref) <= 1e-12 * ref, case
        if shard > valid:  # the padding segment's partial is +0.0
            assert part_a[count - 1].cpu().numpy().view(np.int64) == 0, case


def test_local_share_full_size_rank7_of_llama3_8b_w8(device):
    """Rank 7 of Llama-3-8B at W=8 through ``hbt_grad_local_share_sqnorm``: its slice starts
    7,026,478,592 elements into each rank's padded bf16 gradient, far past 2^31, so every
    offset must be 64-bit.  2^20 sampled outputs and both ends of the shard are checked
    bitwise against numpy on the same eight bf16 values in rank order; the partials'
    sum against torch's fp64 sum of squares of the whole output."""
    lib = _native.library()
    group, shard = 8, 1_003_782_656
    rank = group - 1
    offset = rank * shard
    gen = torch.Generator(device=device).manual_seed(77)
    grads = []
    for _ in range(group):
        g = torch.empty(group * shard, dtype=torch.bfloat16, device=device)  # only rank 7's slice is read
        g[offset:].copy_(torch.randn(shard, device=device, generator=gen).mul_(1e-2))
        grads.append(g)
    out = torch.empty(shard, dtype=torch.float32, device=device)
    chunk = 32768
    partials = torch.empty(-(-shard // chunk), dtype=torch.float64, device=device)
    tile_sums = torch.empty(-(-shard // 256), dtype=torch.float64, device=device)
    status = lib.hbt_grad_local_share_sqnorm(
        _native.pointer_array([g.data_ptr() for g in grads]), group, rank, shard, shard,
        _native.dtype_code(torch.bfloat16), _native.dtype_code(torch.float32), float(group),
        _native.dtype_code(torch.float32), ctypes.c_void_p(out.data_ptr()),
        ctypes.c_void_p(partials.data_ptr()), ctypes.c_void_p(tile_sums.data_ptr()),
        ctypes.c_void_p(_native.stream_of(device)),
    )
    _native.check(status, "test.local_share_full")
    idx = torch.randint(0, shard, (1 << 20,), device=device, generator=gen)
    idx = torch.cat([idx, torch.arange(0, 4096, device=device), torch.arange(shard - 4096, shard, device=device)])
    vals = np.stack([g[offset:][idx].float().cpu().numpy() for g in grads])  # exact widening
    expect = vals[0] / np.float32(group)
    for q in range(1, group):
        expect = (expect + vals[q] / np.float32(group)).astype(np.float32)
    assert np.array_equal(out[idx].cpu().numpy().view(np.int32), expect.view(np.int32))
    ref = float(out.double().pow(2).sum())
    assert abs(float(partials.sum()) - ref) <= 1e-10 * ref
    del grads
    torch.cuda.empty_cache()


def test_local_share_across_two_launch_slices(device):
    """A shard whose tiles do not fit one launch: a HIP grid dimension holds at most
    2^32 - 1 work-items, so 64-lane workgroups split after 67,108,863 tiles of 256
    elements.  A G = 1 local share of 17,180,124,928 bf16 elements (1,000 tiles past the
    limit) runs as two launches, and its tile sums sit in two differently sized
    XCD-grouped slices.  The output must be the exact widening of every element (zeros
    over the padding), and every norm partial must match an independent norm pass over
    the output, chunk by chunk, within 1e-12."""
    torch.cuda.empty_cache()
    free, _ = torch.cuda.mem_get_info(device)
    if free < 120e9:
        pytest.skip(f"needs about 104 GB of free device memory, {free / 1e9:.0f} GB free")
    lib = _native.library()
    slice_tiles = (2**32 - 1) // 64
    shard = (slice_tiles + 1000) * 256
    valid = shard - 1000
    gen = torch.Generator(device=device).manual_seed(91)
    x = torch.randn(shard, dtype=torch.bfloat16, device=device, generator=gen)
    out = torch.empty(shard, dtype=torch.float32, device=device)
    chunk = 32768
    valid_chunks, pad_chunks = -(-valid // chunk), -(-(shard - valid) // chunk)
    partials = torch.empty(valid_chunks + pad_chunks, dtype=torch.float64, device=device)
    tile_sums = torch.empty(-(-shard // 256), dtype=torch.float64, device=device)
    status = lib.hbt_grad_local_share_sqnorm(
        _native.pointer_array([x.data_ptr()]), 1, 0, shard, valid,
        _native.dtype_code(torch.bfloat16), _native.dtype_code(torch.float32), 1.0,
        _native.dtype_code(torch.float32), ctypes.c_void_p(out.data_ptr()),
        ctypes.c_void_p(partials.data_ptr()), ctypes.c_void_p(tile_sums.data_ptr()),
        ctypes.c_void_p(_native.stream_of(device)),
    )
    _native.check(status, "test.local_share_two_slices")
    step = 1 << 30
    for i in range(0, valid, step):
        j = min(valid, i + step)
        assert torch.equal(out[i:j].view(torch.int32), x[i:j].float().view(torch.int32)), i
    assert bool((out[valid:] == 0.0).all())
    del x
    reference = torch.empty_like(partials)
    status = lib.hbt_grad_sqnorm_partials(
        _native.pointer_array([out.data_ptr(), out.data_ptr() + valid * 4]),
        _native.int64_array([valid, shard - valid]), _native.double_array([1.0, 1.0]), 2,
        _native.dtype_code(torch.float32), 1.0, reference.data_ptr(), _native.stream_of(device),
    )
    _native.check(status, "test.sqnorm_two_slices")
    assert bool(((partials - reference).abs() <= 1e-12 * reference.abs()).all())
    assert bool((partials[valid_chunks:] == 0.0).all())
    del out, tile_sums, partials, reference
    torch.cuda.empty_cache()


@pytest.mark.parametrize("acc_dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("assign", [False, True])
def test_grad_accumulate_tiles(device, acc_dtype, grad_dtype, assign):
    """``hbt_grad_accumulate`` (the ``no_sync`` accumulation of ``parallel/fsdp.py:738-749``)
    against torch's CPU ops in the accumulator's dtype: ``acc.add_(grad.to(acc_dtype))``,
    or ``grad.to(acc_dtype)`` itself with ``HBT_ACCUMULATE_ASSIGN`` (the first
    micro-batch's clone).  Bitwise except that NaN results are compared as NaN.  Several
    pairs per launch, tails of every length, a misaligned first pair (scalar path),
    signed zeros, infinities, a NaN and subnormal sums."""
    lib = _native.library()
    gen = torch.Generator(device=device).manual_seed(11)
    sizes = [1, 7, 255, 256, 257, 4097, 100_003]
    acc_base = (torch.randn(sum(sizes) + 1, device=device, generator=gen) * 1e-2).to(acc_dtype)
    grad_base = (torch.randn(sum(sizes) + 1, device=device, generator=gen) * 1e-2).to(grad_dtype)
    acc_base[1:5] = -0.0
    grad_base[1:3] = -0.0     # -0 + -0 = -0
    grad_base[3:5] = 0.0      # -0 + +0 = +0
    acc_base[300] = float("inf")
    grad_base[301] = -float("inf")
    grad_base[302] = float("nan")
    acc_base[303] = torch.finfo(acc_dtype).tiny / 8   # subnormal where the dtype has them
    grad_base[303] = torch.finfo(grad_dtype).tiny
    grad_base[304] = torch.finfo(grad_dtype).max      # overflows a narrower accumulator dtype
    accs, grads, cursor = [], [], 1  # the first pair starts one element in: misaligned
    for n in sizes:
        accs.append(acc_base[cursor:cursor + n])
        grads.append(grad_base[cursor:cursor + n])
        cursor += n
    before = [a.detach().cpu().clone() for a in accs]
    lead = _bits(acc_base[:1])
    stream = ctypes.c_void_p(_native.stream_of(device))
    status = lib.hbt_grad_accumulate(
        _native.pointer_array([a.data_ptr() for a in accs]), _native.pointer_array([g.data_ptr() for g in grads]),
        _native.int64_array(sizes), len(sizes), _native.dtype_code(acc_dtype), _native.dtype_code(grad_dtype),
        _native.ACCUMULATE_ASSIGN if assign else 0, stream,
    )
    _native.check(status, "test.grad_accumulate")
    for a, b, g in zip(accs, before, grads):
        cast = g.detach().cpu().to(acc_dtype)
        expect = cast if assign else b.add_(cast)
        got = a.detach().cpu()
        nan = torch.isnan(expect)
        assert torch.equal(torch.isnan(got), nan)
        assert np.array_equal(_bits(got)[~nan.numpy()], _bits(expect)[~nan.numpy()])
    assert np.array_equal(_bits(acc_base[:1]), lead)  # the element before the first pair is untouched
    if not assign:
        assert bool(torch.signbit(accs[0][0])) and not bool(torch.signbit(accs[1][2]))
    # host-side refusals: no launch
    too_many = _native.MAX_TENSORS_PER_LAUNCH + 1
    assert lib.hbt_grad_accumulate(_native.pointer_array([accs[0].data_ptr()] * too_many),
                                   _native.pointer_array([grads[0].data_ptr()] * too_many),
                                   _native.int64_array([1] * too_many), too_many, _native.dtype_code(acc_dtype),
                                   _native.dtype_code(grad_dtype), 0, stream) == -1
    assert lib.hbt_grad_accumulate(_native.pointer_array([accs[0].data_ptr()]),
                                   _native.pointer_array([grads[0].data_ptr()]), _native.int64_array([1]), 1,
                                   0 if acc_dtype == torch.float64 else _native.dtype_code(acc_dtype), 3, 0,
                                   stream) == -1  # fp64 gradients need an fp64 accumulator
