"""``bench.py`` measures one GPU: any ``--gpus`` other than 1 exits with status 2 and a
message before touching a device, for the headline and every other workload."""

from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("workload", ["adamw", "buckets", "fsdp"])
def test_more_than_one_gpu_is_refused(workload):
    result = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--workload", workload],
                            capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert result.returncode == 2
    assert "--gpus must be 1" in result.stderr
    assert result.stdout == ""
