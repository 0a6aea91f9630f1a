"""Pins the oracle's norm, clip and bf16 restatements.

* ``sqnorm`` against ``math.fsum`` (exactly rounded sums) on inputs where the sum of
  squares is exact in fp64, and against torch's fp64 ``pow(2).sum()`` (the
  reference's own op sequence, ``optim/sharded_optimizer.py:154-158``).
* The reference's known answers: a per-element weight vector ``[2, 2, 1, 0]`` with
  unit gradients at world size 4 gives 1.25
  (``tests/unit/test_single_process_components.py:364-371``), and gradients of 3 over
  4 elements have norm 6 and are clipped to norm 1 (``:397-406``).
* ``f32_to_bf16`` bitwise against ``Tensor.to(torch.bfloat16)`` on specials and random values.
"""

from __future__ import annotations

import math

import numpy as np
import torch

import oracle


def test_sqnorm_against_fsum():
    rng = np.random.default_rng(0)
    for n in (1, 7, 1000, 12345):
        g = (rng.standard_normal(n) * 10.0 ** rng.integers(-6, 3)).astype(np.float32)
        exact = math.fsum(float(x) * float(x) for x in g)
        assert oracle.sqnorm(g) == exact


def test_sqnorm_against_torch_fp64_reduction():
    g = (torch.randn(1 << 20) * 1e-4).numpy()
    ref = float(torch.from_numpy(g).to(torch.float64).pow(2).sum())
    assert abs(oracle.sqnorm(g) - ref) <= 1e-12 * ref


def test_sqnorm_unscale_and_bf16():
    g = np.array([65536.0, -131072.0, 32768.0], dtype=np.float32)
    assert oracle.sqnorm(g, unscale=2.0**-16) == 1.0 + 4.0 + 0.25
    bits = oracle.f32_to_bf16(g)
    assert oracle.sqnorm(bits, unscale=2.0**-16) == 5.25


def test_sqnorm_nonfinite_propagates():
    assert math.isinf(oracle.sqnorm(np.array([1.0, np.inf], np.float32)))
    assert math.isnan(oracle.sqnorm(np.array([np.nan, 1.0], np.float32)))


def test_weighted_known_answer():
    # Per-element weights [2, 2, 1, 0] / world 4 on unit gradients: (2 + 2 + 1 + 0) / 4.
    weights = np.array([2.0, 2.0, 1.0, 0.0]) / 4
    g = np.ones(4, np.float32)
    total = sum(w * oracle.sqnorm(g[i : i + 1]) for i, w in enumerate(weights))
    assert total == 1.25


def test_clip_known_answer():
    g = np.full(4, 3.0, np.float32)
    norm = math.sqrt(oracle.sqnorm(g))
    assert norm == 6.0
    mul = oracle.clip_multiplier(norm, 1.0)
    clipped = (g * np.float32(mul)).astype(np.float32)
    assert abs(math.sqrt(oracle.sqnorm(clipped)) - 1.0) < 1e-5
    assert oracle.clip_multiplier(0.5, 1.0) == 1.0
    assert oracle.clip_multiplier(6.0, 0.0) == 1.0
    assert oracle.clip_multiplier(float("inf"), 1.0) == 0.0
    assert oracle.clip_multiplier(float("nan"), 1.0) == 1.0


def test_clip_matches_reference_mul():
    # The reference multiplies by a Python float: torch rounds it to fp32 once.
    g = torch.randn(1000)
    norm = float(torch.linalg.vector_norm(g.double()))
    coef = 0.37 / (norm + 1e-6)
    expect = g.clone().mul_(coef).numpy()
    got = (g.numpy() * np.float32(oracle.clip_multiplier(norm, 0.37))).astype(np.float32)
    assert np.array_equal(expect, got)


def test_bf16_rounding_against_torch():
    specials = np.array(
        [0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-40, 1.00390625,
         1.01171875, 1.0039062 + 1e-7, 65504.0],
        dtype=np.float32,
    )
    rng = np.random.default_rng(1)
    rand = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32),
        rng.integers(0, 2**32, 100_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
    ])
    rand = rand[~np.isnan(rand)]
    for x in (specials, rand):
        expect = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(oracle.f32_to_bf16(x), expect)
    assert oracle.f32_to_bf16(np.array([np.nan], np.float32))[0] == 0x7FC0
