"""The C-ABI library loads and exports exactly what ``include/hbt.h`` declares.

Runs without a GPU: loading ``libhbt.so`` and querying its constant entry points
issues no device call.
"""

from __future__ import annotations

import os
import re

import pytest

from hybrid_training_amd import _native
from hybrid_training_amd.errors import NativeKernelError, UnsupportedFeatureError

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "hbt.h")


def _declared_functions() -> set[str]:
    text = open(HEADER, encoding="utf-8").read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(hbt_[a-z0-9_]+)\s*\(", text))


def test_header_and_binding_agree():
    declared = _declared_functions()
    assert declared == set(_native.EXPORTED_SYMBOLS), declared ^ set(_native.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.library()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.hbt_abi_version() == _native.ABI_VERSION
    assert lib.hbt_symbol_count() == len(_declared_functions())
    assert lib.hbt_norm_partials_count(_native.int64_array([1, 32768, 32769]), 3, 0) == 1 + 1 + 2
    assert lib.hbt_norm_partials_count(_native.int64_array([1, 65536, 65537]), 3, 1) == 1 + 1 + 2
    assert lib.hbt_norm_partials_count(None, 99, 0) == -1
    assert lib.hbt_norm_partials_count(_native.int64_array([1]), 1, 7) == -1
    # 1 KB of source per chunk
    assert lib.hbt_copy_chunk_elems(0, 0) == 256 and lib.hbt_copy_chunk_elems(1, 1) == 512
    assert lib.hbt_copy_chunk_elems(0, 1) == 256 and lib.hbt_copy_chunk_elems(1, 0) == 512
    assert lib.hbt_copy_chunk_elems(3, 3) == -1
    assert lib.hbt_last_error() == b""


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = _native.library()
    # count out of range: refused on the host, no device touched.
    status = lib.hbt_adamw_step(None, None, None, None, None, 99, 0, 1.0, None,
                                1, 0.1, 0.9, 0.1, 1, 1e-8, -1e-3, None)
    assert status == -1
    assert b"count" in lib.hbt_last_error()
    with pytest.raises(NativeKernelError, match="count"):
        _native.check(status, "test")
    assert lib.hbt_copy_intervals(None, 1, 1, 0, 0, 0, 1.0, 0, None) == -1
    assert lib.hbt_copy_intervals(None, 0, 0, 0, 0, 0, 1.0, 0, None) == 0
    assert lib.hbt_copy_intervals(None, 0, 0, 0, 0, 0, 1.0, 2, None) == -1  # unknown flag
    assert lib.hbt_grad_local_share(None, 0, 0, 1, 1, 0, 1.0, None, None) == -1
    assert lib.hbt_grad_local_share_sqnorm(None, 1, 0, 1, 1, 0, 1.0, None, None, None, None) == -1
    assert b"hbt_grad_local_share_sqnorm" in lib.hbt_last_error()
    assert lib.hbt_grad_norm_finalize(None, 5, 1.0, None, None, None, None, None) == -1


def test_host_tensors_are_refused():
    import torch

    with pytest.raises(UnsupportedFeatureError, match="HIP device"):
        _native.require_device_tensor(torch.zeros(3), "test")
