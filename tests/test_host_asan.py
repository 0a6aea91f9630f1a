"""The library's host code under AddressSanitizer (CPU only, no device).

The C entry points validate their arguments and build their launch tables on the host
before any kernel runs.  This test builds ``libhbt.so`` with AddressSanitizer on the host
code only (``-Xarch_host``; the gfx950 device code is built as usual), links
``tests/host_asan_drive.c`` against it with clang's sanitizer runtime, and runs the drive:
every entry point with tables of every size up to and one past its limit, empty tensors
(nothing to launch) and bad pointers, sizes and dtypes.  Any out-of-bounds or
use-after-free access on the host fails the run; so does an unexpected return code.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from hybrid_training_amd import _native

from .test_native_abi import _declared_functions

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "build-your-own-hybrid-distributed-training_amd", "csrc")
CLANG = "/opt/rocm/llvm/bin/clang"
HOST_ASAN = "-Xarch_host -fsanitize=address -Xarch_host -fno-omit-frame-pointer -g"


def test_host_code_under_address_sanitizer(tmp_path):
    if shutil.which("make") is None or not os.path.exists(CLANG) or shutil.which("hipcc") is None \
            and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("needs make, hipcc and ROCm's clang")
    lib = tmp_path / "libhbt.so"
    build = subprocess.run(["make", "-s", "-B", "-j8", "-C", CSRC, f"OUT={lib}", f"BUILD={tmp_path / 'obj'}",
                            f"EXTRA={HOST_ASAN}"], capture_output=True, text=True, timeout=900)
    assert build.returncode == 0, build.stderr[-2000:]
    exe = tmp_path / "drive"
    link = subprocess.run([CLANG, "-std=c11", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
                           f"-DHBT_TEST_ABI={_native.ABI_VERSION}", f"-DHBT_TEST_SYMBOLS={len(_declared_functions())}",
                           "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "host_asan_drive.c"),
                           "-L", str(tmp_path), "-lhbt", f"-Wl,-rpath,{tmp_path}", "-o", str(exe)],
                          capture_output=True, text=True, timeout=300)
    assert link.returncode == 0, link.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0")
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert "AddressSanitizer" not in run.stderr, run.stderr[-4000:]
    assert run.returncode == 0 and "0 failures" in run.stdout, run.stdout + run.stderr[-2000:]
