"""GPU parity of the interval gather-copy kernel (``hbt_copy_intervals``).

Every case builds the expected destination on the CPU with numpy slicing (and the
oracle's bf16 rounding) and requires bitwise equality: copies are byte work.
Intervals start at arbitrary element offsets on both sides, so the aligned, the
byte-shifted and the head/tail paths all run.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import _native

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    as_int = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
    return t.view(as_int).numpy().copy()


def _as_f32(bits16: np.ndarray) -> np.ndarray:
    return (bits16.astype(np.uint32) << 16).view(np.float32)


def _to_f32(bits: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """fp32 values of element bit patterns (widening is exact for every dtype here)."""
    if dtype == torch.float32:
        return bits.view(np.float32)
    if dtype == torch.float16:
        return bits.view(np.float16).astype(np.float32)
    return _as_f32(bits)


def _from_f32(vals: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Bit patterns of fp32 values rounded to ``dtype`` (round to nearest even)."""
    if dtype == torch.float32:
        return vals.view(np.int32)
    if dtype == torch.float16:
        with np.errstate(over="ignore"):
            return vals.astype(np.float16).view(np.int16)
    return oracle.f32_to_bf16(vals).view(np.int16)


def _converter(sdt, ddt, op, divisor):
    """The expected element map of one plan, on bit patterns."""
    if sdt == ddt and op == _native.COPY_OP_COPY:
        return lambda x: x

    def convert(x):
        vals = _to_f32(x, sdt)
        if op == _native.COPY_OP_DIVIDE:
            vals = (vals / np.float32(divisor)).astype(np.float32)
        return _from_f32(vals, ddt)

    return convert


def _random_intervals(rng, n_src, n_dst, count, max_len):
    """Non-overlapping destination intervals (random order), random source offsets."""
    cuts = np.sort(rng.choice(np.arange(1, n_dst), size=2 * count, replace=False))
    rows = []
    for k in range(count):
        d0, d1 = int(cuts[2 * k]), int(cuts[2 * k + 1])
        n = min(d1 - d0, max_len)
        s0 = int(rng.integers(0, n_src - n))
        rows.append((s0, d0, n))
    rng.shuffle(rows)
    return rows


def _expected(src_vals, dst_init, rows, convert):
    out = dst_init.copy()
    for s0, d0, n in rows:
        out[d0 : d0 + n] = convert(src_vals[s0 : s0 + n])
    return out


CASES = [
    # (src dtype, dst dtype, op)
    (torch.float32, torch.float32, _native.COPY_OP_COPY),
    (torch.bfloat16, torch.bfloat16, _native.COPY_OP_COPY),
    (torch.float16, torch.float16, _native.COPY_OP_COPY),
    (torch.float64, torch.float64, _native.COPY_OP_COPY),
    (torch.float32, torch.bfloat16, _native.COPY_OP_COPY),
    (torch.bfloat16, torch.float32, _native.COPY_OP_COPY),
    (torch.float32, torch.float32, _native.COPY_OP_DIVIDE),
    (torch.bfloat16, torch.bfloat16, _native.COPY_OP_DIVIDE),
    (torch.bfloat16, torch.float32, _native.COPY_OP_DIVIDE),
    (torch.float32, torch.bfloat16, _native.COPY_OP_DIVIDE),
    (torch.float32, torch.float16, _native.COPY_OP_COPY),
    (torch.float16, torch.float32, _native.COPY_OP_COPY),
    (torch.float16, torch.float16, _native.COPY_OP_DIVIDE),
    (torch.float32, torch.float16, _native.COPY_OP_DIVIDE),
    (torch.float16, torch.float32, _native.COPY_OP_DIVIDE),
]


@pytest.mark.parametrize(("sdt", "ddt", "op"), CASES)
@pytest.mark.parametrize("count,max_len", [(7, 100_000), (300, 3_000), (2000, 40)])
def test_random_interval_plans(device, sdt, ddt, op, count, max_len):
    rng = np.random.default_rng(count * 7 + int(op) + 31 * CASES.index((sdt, ddt, op)))
    n_src, n_dst = 400_003, 500_009
    src = (torch.randn(n_src, dtype=torch.float32, device=device) * 3).to(sdt)
    dst = (torch.randn(n_dst, dtype=torch.float32, device=device)).to(ddt)
    dst_init = _bits(dst)
    rows = _random_intervals(rng, n_src, n_dst, count, max_len)
    divisor = 3.0 if op == _native.COPY_OP_DIVIDE else 1.0
    plan = _native.CopyPlan(device)
    for s0, d0, n in rows:
        plan.add(src, s0, dst, d0, n)
    plan.run(src_dtype=sdt, dst_dtype=ddt, op=op, divisor=divisor)
    sbits = _bits(src)
    expect = _expected(sbits, dst_init, rows, _converter(sdt, ddt, op, divisor))
    assert np.array_equal(_bits(dst), expect)


def test_zero_fill_mixed_with_copies(device):
    src = torch.randn(10_000, device=device)
    dst = torch.full((20_000,), 7.0, device=device)
    plan = _native.CopyPlan(device)
    plan.add(src, 1, dst, 3, 5000)
    plan.add_zero(dst, 5003, 1234)
    plan.add_zero(dst, 19_999, 1)
    plan.add(src, 5000, dst, 7001, 4999)
    plan.run(src_dtype=torch.float32, dst_dtype=torch.float32)
    expect = np.full(20_000, 7.0, np.float32)
    s = src.cpu().numpy()
    expect[3:5003] = s[1:5001]
    expect[5003:6237] = 0.0
    expect[19_999] = 0.0
    expect[7001:12_000] = s[5000:9999]
    assert np.array_equal(dst.cpu().numpy().view(np.int32), expect.view(np.int32))


@pytest.mark.parametrize("src_off,dst_off", [(0, 0), (3, 0), (0, 5), (7, 1), (1, 6)])
def test_large_interval_every_alignment(device, src_off, dst_off):
    n = 50_000_000 + 13
    src = torch.randint(-(2**15), 2**15 - 1, (n + 8,), dtype=torch.int16, device=device).view(torch.bfloat16)
    dst = torch.zeros(n + 8, dtype=torch.bfloat16, device=device)
    plan = _native.CopyPlan(device)
    plan.add(src, src_off, dst, dst_off, n)
    plan.run(src_dtype=torch.bfloat16, dst_dtype=torch.bfloat16)
    assert torch.equal(dst[dst_off : dst_off + n].view(torch.int16), src[src_off : src_off + n].view(torch.int16))
    assert int(dst[:dst_off].view(torch.int16).abs().sum()) == 0
    assert int(dst[dst_off + n :].view(torch.int16).abs().sum()) == 0


def test_in_place_divide(device):
    x = torch.randn(1_000_003, device=device)
    expect = (x.cpu().numpy() / np.float32(8.0)).astype(np.float32)
    plan = _native.CopyPlan(device)
    plan.add(x, 0, x, 0, x.numel())
    plan.run(src_dtype=torch.float32, dst_dtype=torch.float32, op=_native.COPY_OP_DIVIDE, divisor=8.0)
    assert np.array_equal(x.cpu().numpy().view(np.int32), expect.view(np.int32))


@pytest.mark.parametrize("divisor", [3.0, 8.0, 0.5, 2.0**-120])
def test_specials_round_trip_and_divide(device, divisor):
    """Specials through the bf16 narrowing and the divide.  Power-of-two divisors take the
    exact-reciprocal multiply and must give the bits of numpy's division, subnormal
    results and overflow to inf included."""
    vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 3.4e38, 1.0, 1.00390625,
                     1.1754944e-38, 3e-45, 1.5e-38, -2.3e-38, 7.0, 1e30], np.float32)
    src = torch.from_numpy(vals).to(device)
    out16 = torch.empty(vals.size, dtype=torch.bfloat16, device=device)
    plan = _native.CopyPlan(device)
    plan.add(src, 0, out16, 0, vals.size)
    plan.run(src_dtype=torch.float32, dst_dtype=torch.bfloat16)
    assert np.array_equal(_bits(out16).view(np.uint16), oracle.f32_to_bf16(vals))
    div = torch.empty_like(src)
    plan = _native.CopyPlan(device)
    plan.add(src, 0, div, 0, vals.size)
    plan.run(src_dtype=torch.float32, dst_dtype=torch.float32, op=_native.COPY_OP_DIVIDE, divisor=divisor)
    with np.errstate(over="ignore", under="ignore"):
        expect = (vals / np.float32(divisor)).astype(np.float32)
    got = div.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(expect))
    assert np.array_equal(got[~np.isnan(got)].view(np.int32), expect[~np.isnan(expect)].view(np.int32))


def test_plan_bounds_are_checked_on_the_host(device):
    a = torch.zeros(10, device=device)
    plan = _native.CopyPlan(device)
    with pytest.raises(ValueError, match="runs past"):
        plan.add(a, 5, a, 0, 6)
    with pytest.raises(ValueError, match="runs past"):
        plan.add_zero(a, 8, 3)


def _element_size(dtype):
    return torch.empty(0, dtype=dtype).element_size()


# The divisor only matters for DIVIDE: a copy runs once, dividing cases with both divisors.
_ALIGNED_CASES = [(sdt, ddt, op, divisor) for sdt, ddt, op in CASES if sdt != torch.float64
                  for divisor in ((3.0, 8.0) if op == _native.COPY_OP_DIVIDE else (3.0,))]


@pytest.mark.parametrize(("sdt", "ddt", "op", "divisor"), _ALIGNED_CASES)
def test_aligned_kernel_matches_general_kernel(device, sdt, ddt, op, divisor):
    """Plans whose records all start aligned run through both kernels of
    ``hbt_copy_intervals`` (flags = HBT_COPY_ALIGNED and flags = 0) and must give the
    same bits as numpy: lengths below one unit, around one chunk, with unit tails, and
    zero-fill records.  Divisor 8 takes the exact-reciprocal multiply, 3 the division."""
    lib = _native.library()
    rng = np.random.default_rng(11 + CASES.index((sdt, ddt, op)))
    ssz, dsz = _element_size(sdt), _element_size(ddt)
    s_code, d_code = _native.dtype_code(sdt), _native.dtype_code(ddt)
    chunk = lib.hbt_copy_chunk_elems(s_code, d_code)
    s_quant = (16 * ssz // max(ssz, dsz)) // ssz  # source elements per aligned step
    d_quant = 16 // dsz
    lengths = [1, 3, 7, 8, 9, chunk - 1, chunk, chunk + 1, 2 * chunk + 5, 100_003, 250_000]
    n_src = 2_000_000
    src = (torch.randn(n_src, dtype=torch.float32, device=device) * 3).to(sdt)
    sbits = _bits(src)
    rows, d_cursor = [], 0
    for k, n in enumerate(lengths * 2):
        d0 = d_cursor + int(rng.integers(0, 4)) * d_quant
        s0 = -1 if k % 5 == 4 else int(rng.integers(0, (n_src - n) // s_quant)) * s_quant
        rows.append((s0, d0, n))
        d_cursor = d0 + n + (-(d0 + n)) % d_quant
    n_dst = d_cursor + 64
    if op != _native.COPY_OP_DIVIDE:
        divisor = 1.0
    outs = []
    hints = _native.COPY_HINTS
    for flags in (_native.COPY_ALIGNED, 0, _native.COPY_ALIGNED | hints, hints):
        dst = torch.full((n_dst,), 5.0, dtype=torch.float32, device=device).to(ddt)
        assert src.data_ptr() % 16 == 0 and dst.data_ptr() % 16 == 0
        flat, first = [], 0
        for s0, d0, n in rows:
            assert d0 + n <= n_dst and s0 + n <= n_src
            s_addr = 0 if s0 < 0 else src.data_ptr() + s0 * ssz
            flat += [s_addr, dst.data_ptr() + d0 * dsz, n, first]
            first += -(-n // chunk)
        if flags & hints:  # the record owning every 256th chunk, after the records
            flat += _native.plan_hints(flat[3::4], first)
        table = torch.tensor(flat, dtype=torch.int64).to(device)
        status = lib.hbt_copy_intervals(table.data_ptr(), len(rows), first, s_code, d_code, op, divisor, flags,
                                        _native.stream_of(device))
        _native.check(status, "test.copy_intervals")
        outs.append(_bits(dst))
    convert = _converter(sdt, ddt, op, divisor)
    expect = _bits(torch.full((n_dst,), 5.0, dtype=torch.float32).to(ddt))
    for s0, d0, n in rows:
        expect[d0 : d0 + n] = 0 if s0 < 0 else convert(sbits[s0 : s0 + n])
    for out in outs:
        assert np.array_equal(out, expect)


def test_float16_specials_match_torch(device):
    """fp32 -> fp16 narrowing and fp16 -> fp32 widening against torch's CPU ``.to``:
    ties to even, the overflow threshold (65520 rounds to inf, 65519 to 65504),
    subnormal results down to 2^-24 and below, and NaN staying NaN."""
    vals = np.array([0.0, -0.0, 1.0, 65504.0, 65519.0, 65520.0, -70000.0, 3.4e38, np.inf, -np.inf, np.nan,
                     2.0**-14, 2.0**-24, 2.0**-25, 1.5 * 2.0**-25, 2.0**-26, -3e-8, 1e-40,
                     1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 2049.0, 2051.0, 0.1, -1e-5], np.float32)
    src = torch.from_numpy(vals).to(device)
    out = torch.empty(vals.size, dtype=torch.float16, device=device)
    plan = _native.CopyPlan(device)
    plan.add(src, 0, out, 0, vals.size)
    plan.run(src_dtype=torch.float32, dst_dtype=torch.float16)
    expect = torch.from_numpy(vals).to(torch.float16)
    got = out.cpu()
    nan = torch.isnan(expect)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(torch.int16), expect[~nan].view(torch.int16))
    # every finite fp16 bit pattern widens exactly
    every = torch.arange(-(2**15), 2**15, dtype=torch.int32).to(torch.int16).view(torch.float16)
    finite = every[torch.isfinite(every)].to(device)
    wide = torch.empty(finite.numel(), dtype=torch.float32, device=device)
    plan = _native.CopyPlan(device)
    plan.add(finite, 0, wide, 0, finite.numel())
    plan.run(src_dtype=torch.float16, dst_dtype=torch.float32)
    assert torch.equal(wide.cpu().view(torch.int32), finite.cpu().to(torch.float32).view(torch.int32))


def test_copy_across_two_launch_slices(device):
    """An interval plan whose chunks do not fit one launch: 64-lane workgroups split after
    67,108,863 chunks, 34,359,737,856 bf16 elements at 512 per chunk.  Two records swap
    the halves of a bf16 buffer 100 chunks longer than that (69 GB each way), so the copy
    runs as two launches and the second finds its records through the hint table from a
    nonzero first chunk.  Every element of both halves is compared bitwise."""
    torch.cuda.empty_cache()
    free, _ = torch.cuda.mem_get_info(device)
    if free < 150e9:
        pytest.skip(f"needs about 138 GB of free device memory, {free / 1e9:.0f} GB free")
    slice_chunks = (2**32 - 1) // 64
    n = (slice_chunks + 100) * 512
    half = n // 2
    src = torch.empty(n, dtype=torch.int16, device=device)
    step = 1 << 30
    gen = torch.Generator(device=device).manual_seed(12)
    for i in range(0, n, step):
        src[i : i + step] = torch.randint(-32768, 32767, (min(step, n - i),), dtype=torch.int16, device=device,
                                          generator=gen)
    dst = torch.empty_like(src)
    plan = _native.CopyPlan(device)
    a, b = src.view(torch.bfloat16), dst.view(torch.bfloat16)
    plan.add(a, 0, b, half, half)
    plan.add(a, half, b, 0, n - half)
    plan.run(src_dtype=torch.bfloat16, dst_dtype=torch.bfloat16)
    torch.cuda.synchronize(device)
    assert torch.equal(dst[half:], src[:half])
    assert torch.equal(dst[: n - half], src[half:])
    del src, dst, a, b, plan
    torch.cuda.empty_cache()


def _f16_nan_rules():
    """The NaN bits of x86 F16C conversions, which torch's vectorised CPU ``.to`` uses:
    widening sets the quiet bit and keeps sign and payload; narrowing sets the quiet bit
    and keeps the sign and the payload's top bits.  ``test_oracle_lowp.py`` pins torch's
    vectorised conversions to these rules on the CPU."""
    from oracle import f16_nan_rules

    return f16_nan_rules()


def test_float16_every_bit_pattern_widens_like_torch(device):
    """All 65,536 fp16 bit patterns through fp16 -> fp32: bitwise torch's conversion for
    every non-NaN, and the quiet-bit rule for all 2,046 NaNs (signalling ones included)."""
    widen, narrow = _f16_nan_rules()
    every = torch.arange(-(2**15), 2**15, dtype=torch.int32).to(torch.int16)
    src = every.view(torch.float16).to(device)
    out = torch.empty(every.numel(), dtype=torch.float32, device=device)
    plan = _native.CopyPlan(device)
    plan.add(src, 0, out, 0, every.numel())
    plan.run(src_dtype=torch.float16, dst_dtype=torch.float32)
    bits16 = every.numpy().astype(np.uint16)
    assert np.array_equal(out.cpu().view(torch.int32).numpy().view(np.uint32), widen(bits16))
    # narrowing NaNs of assorted payloads, signalling and quiet, both signs
    payloads = np.array([0x7F800001, 0x7FC12345, 0xFFC00001, 0x7FBFFFFF, 0xFF812345, 0x7FFFFFFF, 0x7FC00000,
                         0xFFFFE000, 0x7F802000], np.uint32)
    nan32 = torch.from_numpy(payloads.view(np.float32)).to(device)
    half = torch.empty(payloads.size, dtype=torch.float16, device=device)
    plan = _native.CopyPlan(device)
    plan.add(nan32, 0, half, 0, payloads.size)
    plan.run(src_dtype=torch.float32, dst_dtype=torch.float16)
    assert np.array_equal(half.cpu().view(torch.int16).numpy().view(np.uint16), narrow(payloads))


def test_bf16_float16_conversions_are_tensor_to(device):
    """bf16 <-> fp16 convert through the exact fp32 value, as ``Tensor.to`` does: round to
    nearest even, fp16 overflow to +-inf, subnormals kept, signed zeros kept."""
    gen = torch.Generator().manual_seed(6)
    exps = torch.rand(20_011, generator=gen) * 60 - 30
    values = torch.randn(20_011, generator=gen) * torch.pow(2.0, exps)
    values[:8] = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 65504.0, 65520.0, 1e-7, 3e-8])
    for src, dst in ((torch.bfloat16, torch.float16), (torch.float16, torch.bfloat16)):
        a = values.to(src)
        b = torch.full((a.numel() + 3,), 7.0, dtype=dst, device=device)
        plan = _native.CopyPlan(device)
        plan.add(a.to(device), 1, b, 3, a.numel() - 1)  # odd offsets on both sides
        plan.run(src_dtype=src, dst_dtype=dst)
        expect = a[1:].to(dst)
        got = b[3 : 3 + expect.numel()].cpu()
        assert torch.equal(got.view(torch.int16), expect.view(torch.int16)), (src, dst)
        untouched = torch.cat([b[:3], b[3 + expect.numel() :]]).cpu()
        assert torch.equal(untouched, torch.full((4,), 7.0, dtype=dst))
