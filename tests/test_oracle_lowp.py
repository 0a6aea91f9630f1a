"""The oracle's 2-byte arithmetic, pinned against torch's CPU ops.

* AdamW and SGD on bfloat16 / float16 parameters, gradients and state: bitwise equal
  to ``torch.optim.AdamW(foreach=False)`` / ``torch.optim.SGD(foreach=False)`` stepping
  the same CPU tensors, over several steps, with and without weight decay, on both
  branches of torch's lerp, with momentum, dampening and Nesterov.  The reference builds
  exactly these optimizers on its flat shards when mixed precision is off and the model
  is bf16 (``parallel/fsdp.py:379-384``, ``optim/sharded_optimizer.py:111-126``).
* The unscale and clip multiplies on bfloat16 gradients: bitwise equal to torch's
  ``grad.mul_(inverse)`` then ``grad.mul_(coefficient)`` on a bf16 CPU tensor
  (``optim/grad_scaler.py:181-186``, ``optim/sharded_optimizer.py:333-337``), followed
  by the fp32 update of the widened gradient.
* The rounding routines: float16 against numpy's conversion, bfloat16 against torch's.

Planted mistakes fail these checks: dropping the rounding of ``eps`` for a bf16 AdamW,
or rounding the gradient only once for both multiplies (see the last tests).
Runs on any host.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

_TORCH = {"bfloat16": torch.bfloat16, "float16": torch.float16}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def _same(a: np.ndarray, b: np.ndarray, dtype: str) -> bool:
    """Bitwise equal, a NaN matching any NaN (torch's CPU kernels and the restatement
    may set different NaN payload bits)."""
    fa, fb = oracle.from_bits(a, dtype), oracle.from_bits(b, dtype)
    return bool(np.all((a == b) | (np.isnan(fa) & np.isnan(fb))))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("lr,betas,wd,eps", [(1e-3, (0.9, 0.999), 0.01, 1e-8), (3e-4, (0.9, 0.95), 0.0, 1e-3),
                                             (5e-2, (0.3, 0.9), 0.1, 1e-4)])
def test_lowp_adamw_is_torch_adamw_on_2_byte_tensors(dtype, lr, betas, wd, eps):
    """``betas[0] = 0.3`` takes torch's lerp branch for weights >= 0.5.  With eps = 1e-8
    (torch's default) an fp16 exp_avg_sq underflows and eps rounds to 0, so updates go
    to inf / NaN in torch and in the restatement alike; the other eps keep them finite."""
    gen = torch.Generator().manual_seed(11)
    n = 40_000
    p = torch.nn.Parameter((torch.randn(n, generator=gen) * 0.05).to(_TORCH[dtype]))
    opt = torch.optim.AdamW([p], lr=lr, betas=betas, eps=eps, weight_decay=wd, foreach=False)
    pb = _bits(p)
    mb = np.zeros(n, np.uint16)
    vb = np.zeros(n, np.uint16)
    for step in range(1, 6):
        g = (torch.randn(n, generator=gen) * 10 ** -(step % 3 + 1)).to(_TORCH[dtype])
        p.grad = g.clone()
        opt.step()
        scalars = oracle.adamw_scalars(lr=lr, beta1=betas[0], beta2=betas[1], eps=eps, weight_decay=wd,
                                       step=float(step))
        oracle.adamw_step(pb, _bits(g), mb, vb, scalars, dtype=dtype)
        state = opt.state[p]
        assert _same(pb, _bits(p), dtype), f"param, step {step}"
        assert _same(mb, _bits(state["exp_avg"]), dtype), f"exp_avg, step {step}"
        assert _same(vb, _bits(state["exp_avg_sq"]), dtype), f"exp_avg_sq, step {step}"
        if eps != 1e-8 or dtype == "bfloat16":
            assert np.isfinite(oracle.from_bits(pb, dtype)).all()


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("momentum,dampening,nesterov,wd", [(0.0, 0.0, False, 0.0), (0.0, 0.0, False, 1e-2),
                                                           (0.9, 0.0, False, 1e-2), (0.9, 0.1, False, 0.0),
                                                           (0.8, 0.0, True, 5e-3)])
def test_lowp_sgd_is_torch_sgd_on_2_byte_tensors(dtype, momentum, dampening, nesterov, wd):
    """On a tensor whose length is a multiple of 64, every element goes through torch's
    vectorised body (its vector width divides 64 on every x86 build)."""
    gen = torch.Generator().manual_seed(5)
    n = 20_480
    lr = 0.07
    p = torch.nn.Parameter((torch.randn(n, generator=gen) * 0.05).to(_TORCH[dtype]))
    opt = torch.optim.SGD([p], lr=lr, momentum=momentum, dampening=dampening, nesterov=nesterov,
                          weight_decay=wd, foreach=False)
    pb = _bits(p)
    buf = np.zeros(n, np.uint16)
    for step in range(4):
        g = (torch.randn(n, generator=gen) * 1e-2).to(_TORCH[dtype])
        p.grad = g.clone()
        opt.step()
        oracle.sgd_step(pb, _bits(g), buf if momentum else None, lr=lr, momentum=momentum, dampening=dampening,
                        weight_decay=wd, nesterov=nesterov, first=step == 0, dtype=dtype)
        assert _same(pb, _bits(p), dtype), f"param, step {step}"
        if momentum:
            assert _same(buf, _bits(opt.state[p]["momentum_buffer"]), dtype), f"buffer, step {step}"


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_lowp_sgd_remainder_form_is_torchs_scalar_loop(dtype):
    """A one-element tensor goes through torch's scalar remainder loop, where each alpha
    product is rounded to the dtype before the add: the oracle's ``remainder`` form is
    that loop bitwise, and differs from the vectorised body's form on some elements."""
    gen = torch.Generator().manual_seed(8)
    n = 3000
    p0 = (torch.randn(n, generator=gen) * 0.05).to(_TORCH[dtype])
    g0 = (torch.randn(n, generator=gen) * 1e-2).to(_TORCH[dtype])
    scalar_loop = []
    for i in range(n):
        p = torch.nn.Parameter(p0[i : i + 1].clone())
        p.grad = g0[i : i + 1].clone()
        torch.optim.SGD([p], lr=0.07, momentum=0.9, weight_decay=0.01, nesterov=True, foreach=False).step()
        scalar_loop.append(_bits(p)[0])
    remainder, body = _bits(p0).copy(), _bits(p0).copy()
    for out, flag in ((remainder, True), (body, False)):
        oracle.sgd_step(out, _bits(g0), np.zeros(n, np.uint16), lr=0.07, momentum=0.9, weight_decay=0.01,
                        nesterov=True, first=True, dtype=dtype, remainder=flag)
    assert _same(remainder, np.array(scalar_loop, np.uint16), dtype)
    assert not np.array_equal(remainder, body)


@pytest.mark.parametrize("inv_scale,coef", [(1.0 / 1000.0, 0.3167), (2.0 ** -16, 0.7), (1.0, 0.123456)])
def test_bf16_gradient_multiplies_round_like_two_mul_calls(inv_scale, coef):
    """The scaled gradient the oracle writes back is torch's ``mul_(inv).mul_(coef)`` on a
    bf16 tensor, and the fp32 update uses exactly that widened value."""
    gen = torch.Generator().manual_seed(3)
    n = 50_000
    g = (torch.randn(n, generator=gen) * 1e-4 / inv_scale).to(torch.bfloat16)
    unscale = float(np.float32(inv_scale))
    grad_mul = float(np.float32(coef))
    expected = g.clone()
    if inv_scale != 1.0:
        expected.mul_(inv_scale)
    expected.mul_(coef)
    p = (torch.randn(n, generator=gen) * 0.02).numpy()
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    out = np.empty(n, np.uint16)
    scalars = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=1.0)
    got_p = p.copy()
    oracle.adamw_step(got_p, _bits(g), m, v, scalars, unscale=unscale, grad_mul=grad_mul, grad_out=out)
    assert np.array_equal(out, _bits(expected))
    # the update of the widened, rounded gradient: the fp32 oracle on expected.float()
    ref_p = p.copy()
    oracle.adamw_step(ref_p, expected.float().numpy(), np.zeros(n, np.float32), np.zeros(n, np.float32), scalars)
    assert np.array_equal(got_p.view(np.uint32), ref_p.view(np.uint32))
    # and the norm of the unscaled bf16 gradient is the norm of torch's unscaled tensor
    unscaled = g.clone()
    if inv_scale != 1.0:
        unscaled.mul_(inv_scale)
    ref = float(unscaled.double().pow(2).sum())
    assert oracle.sqnorm(_bits(g), unscale=unscale) == pytest.approx(ref, rel=1e-12)


def test_bf16_sgd_gradient_multiplies_round_like_two_mul_calls():
    gen = torch.Generator().manual_seed(4)
    n = 10_000
    g = (torch.randn(n, generator=gen) * 10.0).to(torch.bfloat16)
    expected = g.clone().mul_(1.0 / 1000.0).mul_(0.41)
    out = np.empty(n, np.uint16)
    p = np.zeros(n, np.float32)
    oracle.sgd_step(p, _bits(g), None, lr=0.1, unscale=float(np.float32(1.0 / 1000.0)),
                    grad_mul=float(np.float32(0.41)), grad_out=out)
    assert np.array_equal(out, _bits(expected))
    assert np.array_equal(p, np.float32(-0.1) * expected.float().numpy() + np.float32(0.0))


def test_float16_rounding_is_numpys_and_bfloat16_rounding_is_torchs():
    rng = np.random.default_rng(0)
    exps = rng.uniform(-30, 17, 200_000)
    x = (rng.standard_normal(200_000) * 2.0 ** exps).astype(np.float32)
    specials = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 6.0e-8, 2.98e-8, 2.99e-8,
                         6.1035e-5, 6.1e-5, 1e-7, np.inf, -np.inf, 3.0e38], np.float32)
    x = np.concatenate([x, specials])
    with np.errstate(over="ignore"):
        assert np.array_equal(oracle.to_bits(x, "float16"), x.astype(np.float16).view(np.uint16))
        assert np.array_equal(oracle.from_bits(oracle.to_bits(x, "float16"), "float16"),
                              x.astype(np.float16).astype(np.float32))
    assert np.array_equal(oracle.to_bits(x, "bfloat16"), _bits(torch.from_numpy(x).to(torch.bfloat16)))


def test_planted_mistakes_fail_the_pins():
    """Dropping the bf16 rounding of eps, or applying both multiplies before one
    rounding, gives different bits: the pins above would catch either."""
    gen = torch.Generator().manual_seed(1)
    n = 20_000
    v = (torch.rand(n, generator=gen) * 1e-15).to(torch.bfloat16)  # sqrt(v) / 0.3 comparable to eps
    torch_denom = _bits((v.sqrt() / 0.3).add_(1e-8))
    vv = v.float().numpy()
    r = lambda a: oracle.round_to(a, "bfloat16")  # noqa: E731
    unrounded_eps = oracle.to_bits(r(r(np.sqrt(vv)) / np.float32(0.3)) + np.float32(1e-8), "bfloat16")
    rounded_eps = oracle.to_bits(r(np.sqrt(vv)) / np.float32(0.3), "bfloat16")
    rounded_eps = oracle.to_bits(oracle.from_bits(rounded_eps, "bfloat16") + r(np.float32(1e-8)), "bfloat16")
    assert np.array_equal(rounded_eps, torch_denom)
    assert not np.array_equal(unrounded_eps, torch_denom)
    g = (torch.randn(n, generator=gen) * 50).to(torch.bfloat16)
    two = _bits(g.clone().mul_(1.0 / 1000.0).mul_(0.3167))
    once = oracle.to_bits(g.float().numpy() * np.float32(1.0 / 1000.0) * np.float32(0.3167), "bfloat16")
    assert not np.array_equal(two, once)


def test_f16_nan_rules_are_torchs_vectorised_conversions():
    """The fp16 NaN rules the device conversions are held to are torch's own vectorised
    CPU conversions (whole tensors): every fp16 bit pattern widened, and fp32 NaNs of many
    payloads narrowed, bitwise.  A rule that kept signalling NaNs unquieted, or that
    narrowed every NaN to sign | 0x7E00, fails here."""
    widen, narrow = oracle.f16_nan_rules()
    every = torch.arange(-(2**15), 2**15, dtype=torch.int32).to(torch.int16)
    bits16 = every.numpy().astype(np.uint16)
    torch_wide = every.view(torch.float16).to(torch.float32).view(torch.int32).numpy().view(np.uint32)
    assert np.array_equal(widen(bits16), torch_wide)
    rng = np.random.default_rng(5)
    payloads = rng.integers(1, 1 << 23, 4096).astype(np.uint32)
    nans = (payloads | 0x7F800000) | (rng.integers(0, 2, 4096).astype(np.uint32) << 31)
    torch_narrow = torch.from_numpy(nans.view(np.float32)).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(narrow(nans), torch_narrow)
    # planted: unquieted widening, and a canonical narrowed NaN
    snan = (bits16.astype(np.uint32) & 0x7E00) == 0x7C00
    snan &= (bits16.astype(np.uint32) & 0x01FF) != 0
    assert snan.any() and not np.array_equal(widen(bits16) & ~(snan.astype(np.uint32) << 22), torch_wide)
    canonical = ((nans >> 16) & 0x8000 | 0x7E00).astype(np.uint16)
    assert not np.array_equal(canonical, torch_narrow)
