"""The C-ABI library loads and exports exactly what ``include/hbt.h`` declares.

Runs without a GPU: loading ``libhbt.so`` and querying its constant entry points
issues no device call.
"""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
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


# Entry points that compute on the path; the others are introspection helpers that
# share the comment block of the entry point they serve.
_HELPERS = {"hbt_last_error", "hbt_abi_version", "hbt_symbol_count", "hbt_copy_chunk_elems",
            "hbt_norm_partials_count", "hbt_grid_slices"}
# Entry points with no counterpart in the reference: their comment says so and names
# the callers they serve instead of citing a reference function.
_NO_COUNTERPART = {"hbt_grad_norm_noalloc"}
# Plumbing for work recorded into a HIP graph, also with no reference counterpart.
_GRAPH_PLUMBING = {"hbt_write_words"}


def test_every_entry_point_cites_the_reference_interface_it_replaces():
    """Each compute entry point's comment block names the reference function it
    replaces with a ``file.py:line`` citation."""
    text = open(HEADER, encoding="utf-8").read()
    blocks = re.split(r"/\* -{10,}", text)
    cited = {}
    for block in blocks:
        comment, _, code = block.partition("*/")
        code = re.sub(r"/\*.*?\*/", "", code, flags=re.S)
        for name in re.findall(r"\b(hbt_[a-z0-9_]+)\s*\(", code):
            if name in _NO_COUNTERPART:
                cited[name] = "no counterpart in the reference" in comment and "cannot allocate" in comment
            elif name in _GRAPH_PLUMBING:
                cited[name] = "no counterpart in the reference" in comment and "HIP graph" in comment
            else:
                cited[name] = "Replaces:" in comment and re.search(r"[a-z_/]+\.py:\d+", comment) is not None
    compute = _declared_functions() - _HELPERS
    assert compute <= set(cited), compute - set(cited)
    assert all(cited[name] for name in compute), [name for name in compute if not cited[name]]


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
    # 1 KB of source per chunk; 2 KB for the widening 2-byte -> fp32 copies
    assert lib.hbt_copy_chunk_elems(0, 0) == 256 and lib.hbt_copy_chunk_elems(1, 1) == 512
    assert lib.hbt_copy_chunk_elems(0, 1) == 256 and lib.hbt_copy_chunk_elems(1, 0) == 1024
    assert lib.hbt_copy_chunk_elems(2, 0) == 1024 and lib.hbt_copy_chunk_elems(0, 2) == 256
    assert lib.hbt_copy_chunk_elems(3, 3) == 128  # the float64 AVG divide: 1 KB of source
    assert lib.hbt_copy_chunk_elems(9, 0) == -1
    assert lib.hbt_last_error() == b""


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = _native.library()
    # count out of range: refused on the host, no device touched.
    status = lib.hbt_adamw_step(None, None, None, None, None, 99, 0, 0, 1.0, None,
                                1, 0.1, 0.9, 0.1, 1, 1e-8, -1e-3, 0, None)
    assert status == -1
    assert b"count" in lib.hbt_last_error()
    with pytest.raises(NativeKernelError, match="count"):
        _native.check(status, "test")
    assert lib.hbt_copy_intervals(None, 1, 1, 0, 0, 0, 1.0, 0, None) == -1
    assert lib.hbt_copy_intervals(None, 0, 0, 0, 0, 0, 1.0, 0, None) == 0
    assert lib.hbt_copy_intervals(None, 0, 0, 0, 0, 0, 1.0, 4, None) == -1  # unknown flag
    assert lib.hbt_grad_local_share(None, 0, 0, 1, 1, 0, 0, 1.0, 0, None, None) == -1
    assert lib.hbt_grad_local_share_sqnorm(None, 1, 0, 1, 1, 0, 0, 1.0, 0, None, None, None, None) == -1
    assert b"hbt_grad_local_share_sqnorm" in lib.hbt_last_error()
    assert lib.hbt_grad_accumulate(None, None, None, 0, 0, 0, 0, None) == 0  # empty table
    assert lib.hbt_grad_accumulate(None, None, None, 0, 3, 0, 0, None) == 0  # fp64 accumulator, empty table
    assert lib.hbt_grad_accumulate(None, None, None, 0, 0, 3, 0, None) == -1  # fp64 gradient, fp32 accumulator
    assert b"F32, BF16 or F16" in lib.hbt_last_error()
    assert lib.hbt_grad_accumulate(None, None, None, 0, 5, 0, 0, None) == -1  # unknown accumulator dtype
    # fp64 input with an fp32 reduce dtype: refused by the dtype check, before any pointer is read
    fake = ctypes.c_void_p(4096)
    assert lib.hbt_grad_local_share(_native.pointer_array([4096]), 1, 0, 1, 1, 3, 0, 1.0, 0, fake, None) == -1
    assert b"input dtype 3" in lib.hbt_last_error()
    # a master (output) dtype the kernels do not write
    assert lib.hbt_grad_local_share(_native.pointer_array([4096]), 1, 0, 1, 1, 0, 0, 1.0, 3, fake, None) == -1
    assert b"output (master) dtype 3" in lib.hbt_last_error()
    # optimizer dtype pairs: fp32 parameters with fp16 gradients have no kernel; unknown flags
    assert lib.hbt_adamw_step(None, None, None, None, None, 0, 0, 2, 1.0, None,
                              1, 0.1, 0.9, 0.1, 1, 1e-8, -1e-3, 0, None) == -1
    assert b"dtypes (0, 2)" in lib.hbt_last_error()
    assert lib.hbt_adamw_step(None, None, None, None, None, 0, 1, 1, 1.0, None,
                              1, 0.1, 0.9, 0.1, 1, 1e-8, -1e-3, 1, None) == -1
    assert lib.hbt_sgd_step(None, None, None, None, 0, 2, 2, 1.0, None, 0.0, 0.0, 1.0, -0.1, 32, None) == -1
    assert lib.hbt_sgd_step(None, None, None, None, 0, 2, 2, 1.0, None, 0.0, 0.0, 1.0, -0.1, 16, None) == 0
    # conversions: division is refused for float64 and bf16 <-> fp16 pairs (before the table is read)
    assert lib.hbt_copy_intervals(fake, 1, 1, 3, 0, 1, 2.0, 0, None) == -2
    assert lib.hbt_copy_intervals(fake, 1, 1, 1, 2, 1, 2.0, 0, None) == -2
    assert lib.hbt_copy_chunk_elems(3, 0) == 128 and lib.hbt_copy_chunk_elems(0, 3) == 512
    assert lib.hbt_copy_chunk_elems(1, 3) == 1024 and lib.hbt_copy_chunk_elems(2, 3) == 1024
    assert lib.hbt_copy_chunk_elems(1, 2) == 512 and lib.hbt_copy_chunk_elems(3, 3) == 128
    assert lib.hbt_grad_accumulate(None, None, None, 0, 0, 0, 2, None) == -1  # unknown flag
    assert lib.hbt_grad_accumulate(None, None, None, 1, 0, 0, 0, None) == -1  # null table
    assert lib.hbt_grad_norm_finalize(None, 5, 1.0, None, None, None, None, None, None) == -1
    # float64 steps and scaling: table and flag checks on the host
    assert lib.hbt_adamw_step_f64(None, None, None, None, None, 99, 1.0, None,
                                  1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3, 0, None) == -1
    assert b"hbt_adamw_step_f64" in lib.hbt_last_error()
    assert lib.hbt_adamw_step_f64(None, None, None, None, None, 0, 1.0, None,
                                  1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3, 1, None) == -1  # unknown flag
    assert lib.hbt_adamw_step_f64(None, None, None, None, None, 0, 1.0, None,
                                  1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3, 16, None) == 0  # empty table
    assert lib.hbt_sgd_step_f64(None, None, None, None, 0, 1.0, None, 0.0, 0.0, 1.0, -0.1, 2, None) == -1
    assert lib.hbt_sgd_step_f64(None, None, None, None, 0, 1.0, None, 0.0, 0.0, 1.0, -0.1, 16, None) == 0
    assert lib.hbt_scale_inplace_f64(None, None, 1, 1.0, None, None) == -1
    # float64 gradients: the norm takes unscale 1, the fused unscale and the no-allocation norm refuse them
    assert lib.hbt_grad_sqnorm_partials(_native.pointer_array([4096]), _native.int64_array([1]),
                                        _native.double_array([1.0]), 1, 3, 0.5, fake, None) == -2
    assert lib.hbt_scale_inplace_sqnorm(_native.pointer_array([4096]), _native.int64_array([1]), 1, 3, 0.5,
                                        fake, None, None) == -2
    # 2-byte gradients: the fused unscale needs its piece scratch (refused before any launch)
    assert lib.hbt_scale_inplace_sqnorm(_native.pointer_array([4096]), _native.int64_array([1]), 1, 1, 0.5,
                                        fake, None, None) == -1
    assert lib.hbt_grad_norm_noalloc(_native.pointer_array([4096]), _native.int64_array([1]),
                                     _native.double_array([1.0]), 1, 3, 1.0, 1.0, None, None, None, None, None) == -2
    assert lib.hbt_norm_partials_count(_native.int64_array([16384, 16385]), 2, 3) == 3
    # no-allocation norm: bad table, then a request beyond the static scratch, both refused
    # on the host before the scratch address is looked up or anything is launched
    assert lib.hbt_grad_norm_noalloc(None, None, None, 99, 0, 1.0, 1.0, None, None, None, None, None) == -1
    assert b"count" in lib.hbt_last_error()
    too_many = 32768 * 262144 + 1
    status = lib.hbt_grad_norm_noalloc(_native.pointer_array([4096]), _native.int64_array([too_many]),
                                       _native.double_array([1.0]), 1, 0, 1.0, 1.0, None, None, None, None, None)
    assert status == -2
    assert b"static scratch" in lib.hbt_last_error()
    # slot forms of the steps: a null or misaligned slot, or a bad table, is refused before
    # any launch; an empty table with a slot launches nothing
    adam = (1.0, None, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3)
    assert lib.hbt_adamw_step_slot(None, None, None, None, None, 0, 0, 0, *adam, None, 0, None) == -1
    assert b"hbt_adamw_step_slot" in lib.hbt_last_error() and b"16-byte aligned" in lib.hbt_last_error()
    assert lib.hbt_adamw_step_slot(None, None, None, None, None, 0, 0, 0, *adam, ctypes.c_void_p(4104), 0,
                                   None) == -1
    assert lib.hbt_adamw_step_slot(None, None, None, None, None, 99, 0, 0, *adam, fake, 0, None) == -1
    assert b"hbt_adamw_step_slot: count" in lib.hbt_last_error()
    assert lib.hbt_adamw_step_slot(None, None, None, None, None, 0, 0, 0, *adam, fake, 0, None) == 0
    assert lib.hbt_sgd_step_slot(None, None, None, None, 0, 0, 0, 1.0, None, 0.0, 0.0, 1.0, -0.1, None, 0,
                                 None) == -1
    assert lib.hbt_sgd_step_slot(None, None, None, None, 0, 0, 0, 1.0, None, 0.0, 0.0, 1.0, -0.1, fake, 2,
                                 None) == -1  # FIRST_STEP without MOMENTUM
    assert b"hbt_sgd_step_slot: bad flags" in lib.hbt_last_error()
    assert lib.hbt_adamw_step_f64_slot(None, None, None, None, None, 0, *adam, None, 0, None) == -1
    assert lib.hbt_adamw_step_f64_slot(None, None, None, None, None, 0, *adam, fake, 0, None) == 0
    assert lib.hbt_sgd_step_f64_slot(None, None, None, None, 0, 1.0, None, 0.0, 0.0, 1.0, -0.1, None, 0,
                                     None) == -1
    # the writers check the slot, the dtype and the flags before they launch
    assert lib.hbt_adamw_write_scalars(None, 0, 1.0, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3, None) == -1
    assert lib.hbt_adamw_write_scalars(fake, 3, 1.0, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3, None) == -1
    assert b"param_dtype 3" in lib.hbt_last_error()
    assert lib.hbt_adamw_write_scalars_f64(ctypes.c_void_p(4100), 1.0, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3,
                                           None) == -1
    assert lib.hbt_sgd_write_scalars(fake, 0, 1.0, 0.0, 0.0, 1.0, -0.1, 4, None) == -1  # NESTEROV alone
    assert lib.hbt_sgd_write_scalars(fake, 2, 1.0, 0.0, 0.0, 1.0, -0.1, 64, None) == -1  # unknown flag
    assert lib.hbt_sgd_write_scalars_f64(None, 1.0, 0.0, 0.0, 1.0, -0.1, 0, None) == -1
    assert lib.hbt_sgd_write_scalars_f64(fake, 1.0, 0.0, 0.0, 1.0, -0.1, 64, None) == -1
    words = (ctypes.c_uint32 * 2)(1, 2)
    assert lib.hbt_write_words(None, words, 2, None) == -1
    assert lib.hbt_write_words(ctypes.c_void_p(4098), words, 2, None) == -1  # not 4-byte aligned
    assert b"4-byte aligned" in lib.hbt_last_error()
    assert lib.hbt_write_words(fake, None, 2, None) == -1
    assert lib.hbt_write_words(fake, words, -1, None) == -1
    assert lib.hbt_write_words(None, None, 0, None) == 0  # nothing to write, nothing launched
    # the host formatters check what their writers check
    assert lib.hbt_adamw_scalar_record(None, 0, 1.0, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3) == -1
    assert b"hbt_adamw_scalar_record: the record buffer is null" in lib.hbt_last_error()
    record = (ctypes.c_uint8 * _native.STEP_SLOT_BYTES)()
    assert lib.hbt_adamw_scalar_record(record, 3, 1.0, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3) == -1
    assert b"param_dtype 3" in lib.hbt_last_error()
    assert lib.hbt_sgd_scalar_record(record, 0, 1.0, 0.0, 0.0, 1.0, -0.1, 4) == -1  # NESTEROV alone
    assert lib.hbt_sgd_scalar_record(record, 5, 1.0, 0.0, 0.0, 1.0, -0.1, 0) == -1
    assert lib.hbt_adamw_scalar_record_f64(None, 1.0, 1.0, 0.1, 0.9, 0.1, 1.0, 1e-8, -1e-3) == -1
    assert lib.hbt_sgd_scalar_record_f64(record, 1.0, 0.0, 0.0, 1.0, -0.1, 64) == -1  # unknown flag
    assert bytes(record) == bytes(_native.STEP_SLOT_BYTES)  # a refused call writes nothing


def test_scalar_records_fill_the_slot_and_zero_its_tail():
    """The host formatters launch nothing: each writes the whole slot, the scalars it
    was given (as float32 or float64 bit patterns) and zeros after them."""
    lib = _native.library()
    size = _native.STEP_SLOT_BYTES

    def formatted(call, *args):
        record = (ctypes.c_uint8 * size)(*([0xAB] * size))
        assert call(record, *args) == 0
        return bytes(record)

    adam = (0.99999, 0.1, 0.95, 0.05, 0.6324555, 1e-8, -3e-4)
    for dtype in (0, 1, 2):
        raw = formatted(lib.hbt_adamw_scalar_record, dtype, 0.5, *adam)
        assert raw == formatted(lib.hbt_adamw_scalar_record, dtype, 0.5, *adam)  # deterministic
        values = np.frombuffer(raw, dtype=np.float32)
        # eps is kept rounded to a 2-byte parameter's dtype, as torch rounds it there
        assert all(np.float32(a) in values for a in (adam if dtype == 0 else adam[:5] + adam[6:]))
        assert raw.rstrip(b"\0") != raw and 0xAB not in raw
    raw = formatted(lib.hbt_adamw_scalar_record_f64, 0.5, *adam)
    values = np.frombuffer(raw, dtype=np.float64)
    assert all(a in values for a in adam) and 0.5 in values and 0xAB not in raw
    raw = formatted(lib.hbt_sgd_scalar_record, 0, 1.0, 0.01, 0.9, 1.0, -0.1, int(_native.SGD_MOMENTUM))
    assert np.float32(-0.1) in np.frombuffer(raw, dtype=np.float32) and 0xAB not in raw
    raw = formatted(lib.hbt_sgd_scalar_record_f64, 1.0, 0.01, 0.9, 1.0, -0.1, int(_native.SGD_MOMENTUM))
    assert -0.1 in np.frombuffer(raw, dtype=np.float64) and 0xAB not in raw


def test_host_tensors_are_refused():
    import torch

    with pytest.raises(UnsupportedFeatureError, match="HIP device"):
        _native.require_device_tensor(torch.zeros(3), "test")


_C_HOST = r"""
#include <stdio.h>
#include <string.h>
#include "hbt.h"

int main(void) {
    int failures = 0;
    if (hbt_abi_version() != %(abi)d) { printf("abi %%d\n", hbt_abi_version()); failures++; }
    if (hbt_symbol_count() != %(symbols)d) { printf("symbols %%d\n", hbt_symbol_count()); failures++; }
    if (hbt_copy_chunk_elems(HBT_DTYPE_F32, HBT_DTYPE_F32) != 256) failures++;
    if (hbt_copy_chunk_elems(HBT_DTYPE_BF16, HBT_DTYPE_F32) != 1024) failures++;
    /* refused on the host before any device work: a null table with records */
    if (hbt_copy_intervals(NULL, 1, 1, HBT_DTYPE_F32, HBT_DTYPE_F32, HBT_COPY_OP_COPY, 1.0f, 0, NULL)
        != HBT_ERR_INVALID_ARGUMENT) failures++;
    if (strstr(hbt_last_error(), "hbt_copy_intervals") == NULL) failures++;
    if (hbt_adamw_step(NULL, NULL, NULL, NULL, NULL, HBT_MAX_TENSORS_PER_LAUNCH + 1, HBT_DTYPE_F32, HBT_DTYPE_F32,
                       1.0f, NULL, 1.0f, 0.1f, 0.9f, 0.1f, 1.0f, 1e-8f, -1e-3f, HBT_STEP_WRITE_GRAD, NULL)
        != HBT_ERR_INVALID_ARGUMENT)
        failures++;
    {
        int64_t first[3], count[3];
        if (hbt_grid_slices(70000000, 64, first, count, 3) != 2 || first[1] != 67108863 || count[0] != 67108863)
            failures++;
    }
    printf("c host: %%d failures\n", failures);
    return failures;
}
"""


def test_c_host_compiles_against_the_header_and_links(tmp_path):
    """A plain C host (gcc, no HIP headers) includes ``include/hbt.h``, links ``libhbt.so``
    and makes the calls that need no device: the header is valid C and matches the
    library's exports, argument order included."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    lib = _native.library()  # builds the checks above only against a present library
    src = tmp_path / "host.c"
    src.write_text(_C_HOST % {"abi": _native.ABI_VERSION, "symbols": len(_declared_functions())})
    exe = tmp_path / "host"
    libdir = os.path.dirname(_native.library_path())
    subprocess.run([gcc, "-std=c11", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src),
                    "-L", libdir, "-lhbt", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stdout + run.stderr
    assert lib.hbt_abi_version() == _native.ABI_VERSION
