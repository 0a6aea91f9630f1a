"""GPU parity of the flat-buffer helpers (``utils/tensors.py:199-344``).

The cases are the reference's own (``tests/unit/test_tensor_utils.py:51-61``,
``:109-135``) run on the device through the interval copy, plus bf16, non-contiguous
and misaligned inputs: flatten/unflatten is a bitwise round trip, padding rounds up to
the next multiple and no further with exact zeros, an aligned buffer is returned
itself, and bad arguments raise the reference's errors.
"""

from __future__ import annotations

import pytest
import torch

from hybrid_training_amd import ShardingError, build_flat_layout, flatten_dense_tensors, pad_flat_tensor
from hybrid_training_amd import unflatten_to_views

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().cpu().contiguous()
    return t.view({2: torch.int16, 4: torch.int32}[t.element_size()])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_flatten_unflatten_is_lossless(device, dtype):
    gen = torch.Generator(device=device).manual_seed(4)
    wide = torch.randn(5, 7, device=device, generator=gen).to(dtype)
    originals = [torch.randn(2, 3, device=device, generator=gen).to(dtype),
                 torch.randn(4, device=device, generator=gen).to(dtype),
                 wide.t(),                                   # non-contiguous
                 torch.randn(3, 2, device=device, generator=gen).to(dtype)]
    entries, total = build_flat_layout([(f"p{i}", t) for i, t in enumerate(originals)])
    flat = flatten_dense_tensors(originals)
    assert flat.numel() == total == 6 + 4 + 35 + 6
    expect = torch.cat([t.reshape(-1) for t in originals])
    assert torch.equal(_bits(flat), _bits(expect))
    for original, view in zip(originals, unflatten_to_views(flat, entries)):
        assert view.shape == original.shape
        assert torch.equal(_bits(view), _bits(original))
        assert view.data_ptr() >= flat.data_ptr()            # views alias the flat buffer
    out = torch.full((total + 1,), 7.0, device=device).to(dtype)
    again = flatten_dense_tensors(originals, out=out[1:])    # misaligned destination
    assert again.data_ptr() == out[1:].data_ptr()
    assert torch.equal(_bits(again), _bits(expect)) and float(out[0]) == 7.0
    with pytest.raises(ShardingError, match="wrong size"):
        flatten_dense_tensors(originals, out=out)
    with pytest.raises(ShardingError, match="share dtype and device"):
        flatten_dense_tensors([originals[0], originals[1].float() if dtype != torch.float32 else originals[1].half()])
    with pytest.raises(ShardingError, match="nothing to flatten"):
        flatten_dense_tensors([])


@pytest.mark.parametrize(("numel", "multiple", "expected"), [(10, 4, 12), (8, 4, 8), (1, 3, 3), (7, 1, 7), (0, 4, 0)])
def test_pad_to_multiple(device, numel, multiple, expected):
    padded = pad_flat_tensor(torch.ones(numel, device=device), multiple)
    assert padded.numel() == expected
    assert float(padded[:numel].sum()) == numel and float(padded[numel:].abs().sum()) == 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_padding_is_exact_zero_and_aligned_input_is_returned(device, dtype):
    base = torch.full((6,), -3.5, device=device).to(dtype)
    padded = pad_flat_tensor(base[1:], 4)                    # 5 elements, one element into the storage
    assert padded.numel() == 8
    assert torch.equal(_bits(padded[:5]), _bits(base[1:]))
    assert torch.equal(_bits(padded[5:]), torch.zeros(3, dtype=_bits(padded).dtype))  # +0.0, not -0.0
    original = torch.ones(8, device=device).to(dtype)
    assert pad_flat_tensor(original, 4) is original


def test_padding_invalid_arguments(device):
    with pytest.raises(ShardingError, match="one-dimensional"):
        pad_flat_tensor(torch.ones(2, 2, device=device), 4)
    with pytest.raises(ShardingError, match="alignment multiple must be positive"):
        pad_flat_tensor(torch.ones(4, device=device), 0)
    with pytest.raises(ShardingError, match="only zero padding"):
        pad_flat_tensor(torch.ones(5, device=device), 4, value=1.0)
