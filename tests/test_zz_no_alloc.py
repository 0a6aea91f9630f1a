"""``hbt_grad_norm_noalloc`` against ``hbt_grad_sqnorm_partials`` + ``hbt_grad_norm_finalize``.

The no-allocation entry point keeps its norm partials in a static device array; the
workspace pair keeps them in a caller tensor.  Both run the same kernels in the same
order, so every output (fp64 sum, norm, fp32 clip multiplier, non-finite flag) must be
bitwise equal.  Two calls in a row, the second on a smaller input, check that the
array's leftover contents from the first call do not leak into the second.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from hybrid_training_amd import _native

pytestmark = pytest.mark.gpu


def _outputs(device):
    return (torch.full((1,), -1.0, dtype=torch.float64, device=device),
            torch.full((1,), -1.0, dtype=torch.float64, device=device),
            torch.full((1,), -1.0, dtype=torch.float32, device=device),
            torch.full((1,), -1, dtype=torch.int32, device=device))


def _run_workspace(lib, grads, weights, dtype_code, unscale, max_norm, device):
    numels = [int(g.numel()) for g in grads]
    count = int(lib.hbt_norm_partials_count(_native.int64_array(numels), len(grads), dtype_code))
    partials = torch.empty(max(1, count), dtype=torch.float64, device=device)
    stream = _native.stream_of(device)
    _native.check(lib.hbt_grad_sqnorm_partials(
        _native.pointer_array([g.data_ptr() for g in grads]), _native.int64_array(numels),
        _native.double_array(weights), len(grads), dtype_code, unscale, partials.data_ptr(), stream),
        "hbt_grad_sqnorm_partials")
    out = _outputs(device)
    _native.check(lib.hbt_grad_norm_finalize(partials.data_ptr(), count, max_norm, out[0].data_ptr(),
                                             out[1].data_ptr(), out[2].data_ptr(), None, out[3].data_ptr(), stream),
                  "hbt_grad_norm_finalize")
    return out


def _run_noalloc(lib, grads, weights, dtype_code, unscale, max_norm, device):
    numels = [int(g.numel()) for g in grads]
    out = _outputs(device)
    _native.check(lib.hbt_grad_norm_noalloc(
        _native.pointer_array([g.data_ptr() for g in grads]), _native.int64_array(numels),
        _native.double_array(weights), len(grads), dtype_code, unscale, max_norm,
        out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), out[3].data_ptr(), _native.stream_of(device)),
        "hbt_grad_norm_noalloc")
    return out


def _bits(t: torch.Tensor) -> np.ndarray:
    a = t.cpu().numpy()
    return a.view({8: np.uint64, 4: np.uint32}[a.itemsize])


def _assert_same(a, b):
    for x, y in zip(a, b):
        assert np.array_equal(_bits(x), _bits(y)), (x, y)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_norm_matches_the_workspace_pair_on_two_calls(device, dtype):
    lib = _native.library()
    code = _native.dtype_code(dtype)
    gen = torch.Generator(device=device).manual_seed(7)
    # First call: several tensors over many chunks (4.2 M fp32 elements: 129 fp32
    # partials, ragged tails, a misaligned tensor start through a view).
    big = [torch.randn(n, device=device, generator=gen).mul_(1e-2).to(dtype)
           for n in (3_000_001, 1_000_000, 37, 65536 * 3 + 5)]
    big[1] = big[1][1:]  # starts 1 element in: the kernel's scalar path
    weights = [1.0, 0.5, 2.0, 0.125]
    for unscale, max_norm in ((1.0, 1.0), (1.0 / 1000.0, 0.5), (1.0, 0.0)):
        ref = _run_workspace(lib, big, weights, code, unscale, max_norm, device)
        got = _run_noalloc(lib, big, weights, code, unscale, max_norm, device)
        torch.cuda.synchronize()
        _assert_same(got, ref)
    # Second call, smaller: fewer partials than the first call left in the scratch.
    small = [torch.randn(n, device=device, generator=gen).to(dtype) for n in (1000, 5)]
    ref = _run_workspace(lib, small, [1.0, 1.0], code, 1.0, 1.0, device)
    got = _run_noalloc(lib, small, [1.0, 1.0], code, 1.0, 1.0, device)
    torch.cuda.synchronize()
    _assert_same(got, ref)
    assert float(got[0]) == pytest.approx(sum(float(t.double().pow(2).sum()) for t in small), rel=1e-12)
    # An empty call: sum 0, multiplier 1, flag 0.
    got = _run_noalloc(lib, [], [], code, 1.0, 1.0, device)
    torch.cuda.synchronize()
    assert float(got[0]) == 0.0 and float(got[1]) == 0.0 and float(got[2]) == 1.0 and int(got[3]) == 0


def test_noalloc_norm_flags_nonfinite_and_refuses_oversize(device):
    lib = _native.library()
    g = torch.ones(100_000, device=device)
    g[12345] = float("inf")
    ref = _run_workspace(lib, [g], [1.0], 0, 1.0, 1.0, device)
    got = _run_noalloc(lib, [g], [1.0], 0, 1.0, 1.0, device)
    torch.cuda.synchronize()
    _assert_same(got, ref)
    assert int(got[3]) == 1
    # More partials than the static array holds: refused before any launch.
    too_many = 32768 * 262144 + 1
    status = lib.hbt_grad_norm_noalloc(_native.pointer_array([g.data_ptr()]), _native.int64_array([too_many]),
                                       _native.double_array([1.0]), 1, 0, 1.0, 1.0,
                                       None, None, None, None, _native.stream_of(device))
    assert status == -2
    assert b"static scratch" in lib.hbt_last_error()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_norm_allocates_no_device_memory(device, dtype):
    """The entry point takes no device memory of its own: after one warm-up call (which looks
    up the static array's address and lets the runtime set up the launches), repeated calls
    on inputs of different sizes leave the device's free memory (``hipMemGetInfo``, read by
    ``torch.cuda.mem_get_info``) exactly where it was."""
    lib = _native.library()
    code = _native.dtype_code(dtype)
    gen = torch.Generator(device=device).manual_seed(11)
    inputs = [[torch.randn(n, device=device, generator=gen).to(dtype) for n in sizes]
              for sizes in ((2_000_003, 65536 * 5), (1000,), (17, 4097, 300_000))]
    out = _outputs(device)
    numels = [[int(g.numel()) for g in grads] for grads in inputs]
    ptrs = [_native.pointer_array([g.data_ptr() for g in grads]) for grads in inputs]
    sizes = [_native.int64_array(n) for n in numels]
    weights = [_native.double_array([1.0] * len(n)) for n in numels]
    stream = _native.stream_of(device)

    def call(k):
        _native.check(lib.hbt_grad_norm_noalloc(ptrs[k], sizes[k], weights[k], len(numels[k]), code, 1.0, 1.0,
                                                out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(),
                                                out[3].data_ptr(), stream), "hbt_grad_norm_noalloc")

    call(0)
    torch.cuda.synchronize(device)
    free_before, _ = torch.cuda.mem_get_info(device)
    for _ in range(3):
        for k in range(len(inputs)):
            call(k)
    torch.cuda.synchronize(device)
    free_after, _ = torch.cuda.mem_get_info(device)
    assert free_after == free_before
