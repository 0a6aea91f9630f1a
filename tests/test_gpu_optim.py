"""GPU parity of the fused AdamW step and the deterministic norm/clip.

The HIP kernels are called through the C ABI (directly, and through
``ShardedOptimizer``) and compared with the oracle:

* AdamW: bitwise equal to ``oracle.adamw_step`` (both use correctly rounded sqrt
  and division, and the same two fused multiply-adds), across sizes that exercise
  the vector tiles, the tile tail, unaligned views, bf16 gradients, loss-scale and
  clip multipliers, and more tensors than one launch holds.
* AdamW against torch.optim.AdamW on the CPU (the reference's optimizer): within
  ``|a - b| <= 1e-6 * max(|b|, lr)`` per element after 10 steps.
* Norm: within 1e-12 relative of the compensated oracle sum, bitwise reproducible
  run to run, non-finite whenever an element is, and the clip multiplier exactly
  ``fp32(max_norm / (norm + 1e-6))`` of the device norm.
* Full size (one Llama-3-8B FSDP rank at W=8: 1,003,782,656 elements): the
  update checked bitwise on a random subset of 2^20 elements (AdamW is
  element-wise, so a subset check is exact), the norm against torch's fp64 sum.
"""

from __future__ import annotations

import copy
import math

import numpy as np
import pytest
import torch

import oracle
from hybrid_training_amd import GroupHandle, OptimizerConfig, ShardedOptimizer, ShardingError, _native
from hybrid_training_amd.optim import PENDING_UNSCALE_ATTR, gradient_norm_pass

pytestmark = pytest.mark.gpu

RTOL = 1e-6
LLAMA_SHARD = 1_003_782_656  # 8,030,261,248 / 8


def _adamw_launch(ps, gs, ms, vs, scalars, *, unscale=1.0, grad_mul=None):
    lib = _native.library()
    status = lib.hbt_adamw_step(
        _native.pointer_array([t.data_ptr() for t in ps]),
        _native.pointer_array([t.data_ptr() for t in gs]),
        _native.pointer_array([t.data_ptr() for t in ms]),
        _native.pointer_array([t.data_ptr() for t in vs]),
        _native.int64_array([t.numel() for t in ps]),
        len(ps),
        _native.dtype_code(ps[0].dtype),
        _native.dtype_code(gs[0].dtype),
        unscale,
        None if grad_mul is None else grad_mul.data_ptr(),
        *scalars,
        0,
        _native.stream_of(ps[0].device),
    )
    _native.check(status, "test.hbt_adamw_step")


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int32).numpy()


@pytest.mark.parametrize("n", [1, 3, 2047, 2048, 2049, 4096 * 3 + 5, 1 << 20])
def test_adamw_kernel_bitwise_vs_oracle(device, n):
    gen = torch.Generator(device=device).manual_seed(n)
    p = torch.randn(n, device=device, generator=gen) * 0.02
    m = torch.zeros(n, device=device)
    v = torch.zeros(n, device=device)
    P, M, V = p.cpu().numpy(), m.cpu().numpy(), v.cpu().numpy()
    mul = torch.tensor([0.3157], dtype=torch.float32, device=device)
    for step in range(1, 6):
        g = torch.randn(n, device=device, generator=gen) * 1e-3
        sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1,
                                  step=float(step))
        _adamw_launch([p], [g], [m], [v], sc, grad_mul=mul if step % 2 else None)
        oracle.adamw_step(P, g.cpu().numpy(), M, V, sc, grad_mul=0.3157 if step % 2 else 1.0)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(p), P.view(np.int32)), f"param, step {step}"
        assert np.array_equal(_bits(m), M.view(np.int32)), f"exp_avg, step {step}"
        assert np.array_equal(_bits(v), V.view(np.int32)), f"exp_avg_sq, step {step}"


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_adamw_unaligned_views(device, offset):
    n = 10_000
    base = [torch.randn(n + 4, device=device) * s for s in (0.02, 1e-3, 1e-4, 1e-6)]
    base[3] = base[3].abs()
    p, g, m, v = (b[offset : offset + n] for b in base)
    P, G, M, V = (t.cpu().numpy().copy() for t in (p, g, m, v))
    outside = [torch.cat([b[:offset], b[offset + n :]]).cpu() for b in base]
    sc = oracle.adamw_scalars(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, step=3.0)
    _adamw_launch([p], [g], [m], [v], sc)
    oracle.adamw_step(P, G, M, V, sc)
    assert np.array_equal(_bits(p), P.view(np.int32))
    assert np.array_equal(_bits(m), M.view(np.int32))
    assert np.array_equal(_bits(v), V.view(np.int32))
    # Elements outside the views are untouched.
    for b, before in zip(base, outside):
        assert torch.equal(torch.cat([b[:offset], b[offset + n :]]).cpu(), before)


def test_adamw_bf16_grads_with_unscale(device):
    n = 70_001
    g32 = torch.randn(n, device=device) * 1e-4 * 65536
    g16 = g32.to(torch.bfloat16)
    p = torch.randn(n, device=device) * 0.02
    m = torch.randn(n, device=device) * 1e-4
    v = torch.rand(n, device=device) * 1e-8
    P, M, V = p.cpu().numpy(), m.cpu().numpy(), v.cpu().numpy()
    G = g16.cpu().view(torch.int16).numpy().view(np.uint16)
    mul = torch.tensor([0.5], dtype=torch.float32, device=device)
    sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=7.0)
    _adamw_launch([p], [g16], [m], [v], sc, unscale=2.0**-16, grad_mul=mul)
    oracle.adamw_step(P, G, M, V, sc, unscale=2.0**-16, grad_mul=0.5)
    assert np.array_equal(_bits(p), P.view(np.int32))
    assert np.array_equal(_bits(m), M.view(np.int32))
    assert np.array_equal(_bits(v), V.view(np.int32))


@pytest.mark.parametrize("grad_dtype", [torch.float32, torch.bfloat16])
def test_adamw_with_ieee_specials_matches_oracle(device, grad_dtype):
    """IEEE specials through the fused update: gradients +inf, -inf, NaN, -0.0, the
    largest finite value and a denormal, parameters -0.0 and NaN, exp_avg_sq +inf, over
    a vector body and a tail, with and without a clip multiplier: every non-NaN result
    bitwise the oracle's (torch's single-tensor AdamW restated), NaNs in the same places."""
    n = 4096 + 37
    gen = torch.Generator(device=device).manual_seed(71)
    p = torch.randn(n, device=device, generator=gen) * 0.02
    g = torch.randn(n, device=device, generator=gen) * 1e-3
    m = torch.randn(n, device=device, generator=gen) * 1e-4
    v = torch.rand(n, device=device, generator=gen) * 1e-8
    big = torch.finfo(torch.float32).max if grad_dtype == torch.float32 else torch.finfo(torch.bfloat16).max
    for base in (0, 4096):  # the vector body and the tail
        g[base + 0] = float("inf")
        g[base + 1] = -float("inf")
        g[base + 2] = float("nan")
        g[base + 3] = -0.0
        g[base + 4] = big
        g[base + 5] = 1e-40
        p[base + 6] = -0.0
        p[base + 7] = float("nan")
        v[base + 8] = float("inf")
    g = g.to(grad_dtype)
    G = g.cpu().view(torch.int16).numpy().view(np.uint16) if grad_dtype == torch.bfloat16 else g.cpu().numpy()
    for mul in (None, 0.25):
        pp, mm, vv = p.clone(), m.clone(), v.clone()
        P, M, V = pp.cpu().numpy(), mm.cpu().numpy(), vv.cpu().numpy()
        sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=3.0)
        grad_mul = None if mul is None else torch.tensor([mul], dtype=torch.float32, device=device)
        _adamw_launch([pp], [g], [mm], [vv], sc, grad_mul=grad_mul)
        oracle.adamw_step(P, G, M, V, sc, grad_mul=1.0 if mul is None else mul)
        for got, want, what in ((pp, P, "param"), (mm, M, "exp_avg"), (vv, V, "exp_avg_sq")):
            got = got.cpu().numpy()
            nan = np.isnan(want)
            assert np.array_equal(np.isnan(got), nan), (what, mul)
            assert np.array_equal(got[~nan].view(np.int32), want[~nan].view(np.int32)), (what, mul)


def _norm_of(tensors, weights, device, max_norm=0.0):
    segments = [(t, 0, t.numel(), w) for t, w in zip(tensors, weights)]
    return gradient_norm_pass(segments, device, max_norm=max_norm)


@pytest.mark.parametrize("n", [1, 1023, 4096 * 4, 4096 * 4 + 1, 3_000_001])
def test_norm_vs_oracle_and_deterministic(device, n):
    g = torch.randn(n, device=device) * 1e-4
    r1 = _norm_of([g], [1.0], device, max_norm=1e-3)
    r2 = _norm_of([g], [1.0], device, max_norm=1e-3)
    ref = oracle.sqnorm(g.cpu().numpy())
    s1 = float(r1.sum)
    assert abs(s1 - ref) <= 1e-12 * ref
    assert float(r1.norm) == math.sqrt(s1)
    assert torch.equal(r1.sum, r2.sum) and torch.equal(r1.grad_mul, r2.grad_mul)
    expect_mul = oracle.clip_multiplier(float(r1.norm), 1e-3)
    assert float(r1.grad_mul) == expect_mul
    assert int(r1.nonfinite) == 0


def test_norm_weighted_segments_and_known_answer(device):
    # The reference's known answer: weights [2, 2, 1, 0] / 4 over unit gradients -> 1.25.
    g = torch.ones(4, device=device)
    segments = [(g, 0, 2, 0.5), (g, 2, 1, 0.25), (g, 3, 1, 0.0)]
    assert float(gradient_norm_pass(segments, device, max_norm=0.0).sum) == 1.25
    # Many tensors (more than one launch holds), mixed weights.
    tensors = [torch.randn(1000 + 37 * i, device=device) for i in range(21)]
    weights = [1.0 / (1 + i % 3) for i in range(21)]
    got = float(_norm_of(tensors, weights, device).sum)
    ref = sum(w * oracle.sqnorm(t.cpu().numpy()) for t, w in zip(tensors, weights))
    assert abs(got - ref) <= 1e-12 * ref


def test_norm_nonfinite(device):
    g = torch.randn(100_000, device=device)
    g[77_777] = float("inf")
    r = _norm_of([g], [1.0], device, max_norm=1.0)
    assert math.isinf(float(r.norm)) and int(r.nonfinite) == 1
    assert float(r.grad_mul) == 0.0  # coef = 1 / (inf + 1e-6) = 0 < 1, as the reference computes
    g[5] = float("nan")
    r = _norm_of([g], [1.0], device, max_norm=1.0)
    assert math.isnan(float(r.norm)) and int(r.nonfinite) == 1
    assert float(r.grad_mul) == 1.0  # NaN < 1 is false: no clip
    # A non-finite value under weight 0 still poisons the sum (0 * inf = NaN in the reference).
    h = torch.ones(8, device=device)
    h[7] = float("inf")
    r = gradient_norm_pass([(h, 0, 7, 1.0), (h, 7, 1, 0.0)], device, max_norm=0.0)
    assert int(r.nonfinite) == 1


def _make_optimizer(params, lr=3e-4, betas=(0.9, 0.95), wd=0.1, defer=False, in_step=False):
    return ShardedOptimizer(
        params,
        OptimizerConfig(name="adamw", learning_rate=lr, betas=betas, weight_decay=wd, eps=1e-8),
        norm_group=GroupHandle.trivial(),
        device=params[0].device,
        defer_clip=defer,
        clip_in_step=in_step,
    )


def test_sharded_optimizer_vs_torch_adamw(device):
    n, lr, max_norm = 1 << 20, 3e-4, 1.0
    p0 = torch.randn(n) * 0.02
    param = torch.nn.Parameter(p0.to(device))
    opt = _make_optimizer([param], lr=lr)
    ref = torch.nn.Parameter(p0.clone())
    ref_opt = torch.optim.AdamW([ref], lr=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                                foreach=False)
    P, M, V = p0.numpy().copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    worst = 0.0
    gen = torch.Generator().manual_seed(3)
    for step in range(1, 11):
        g = torch.randn(n, generator=gen) * 1e-2  # norm ~ 10: clipping active
        param.grad = g.to(device)
        norm = opt.clip_grad_norm(max_norm)
        opt.step()
        # reference: fp64 norm, python-double coefficient, in-place fp32 multiply, torch AdamW
        ref.grad = g.clone()
        ref_norm = float(g.to(torch.float64).pow(2).sum().sqrt())
        coef = max_norm / (ref_norm + 1e-6)
        if coef < 1.0:
            ref.grad.mul_(coef)
        ref_opt.step()
        assert abs(float(norm) - ref_norm) <= 1e-12 * ref_norm
        # oracle with the device's own multiplier: bitwise
        mul = oracle.clip_multiplier(float(norm), max_norm)
        sc = oracle.adamw_scalars(lr=lr, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1,
                                  step=float(step))
        oracle.adamw_step(P, g.numpy(), M, V, sc, grad_mul=mul)
        got = param.detach().cpu().numpy()
        assert np.array_equal(got.view(np.int32), P.view(np.int32)), f"step {step}"
        want = ref.detach().numpy()
        worst = max(worst, float(np.max(np.abs(got - want) / np.maximum(np.abs(want), lr))))
    assert worst <= RTOL, worst
    state = opt.inner.state[param]
    assert float(state["step"]) == 10.0
    assert torch.equal(state["exp_avg"].cpu(), torch.from_numpy(M))


def test_clip_is_in_place_like_the_reference(device):
    """By default ``clip_grad_norm`` clips .grad in place before it returns, as the
    reference's ``grad.mul_`` does.  With ``clip_in_step`` the step's fused pass writes the
    clipped gradient back instead (or ``materialize_pending`` at once); with
    ``defer_clip`` .grad stays unclipped.  All four give the same parameters."""
    expect = torch.full((4,), 3.0).mul_(1.0 / (6.0 + 1e-6))
    unclipped = torch.full((4,), 3.0)
    results = {}
    for mode in ("eager", "write_back", "materialize", "defer"):
        param = torch.nn.Parameter(torch.ones(4, device=device))
        param.grad = torch.full((4,), 3.0, device=device)
        opt = _make_optimizer([param], defer=(mode == "defer"), in_step=mode in ("write_back", "materialize"))
        before = param.grad._version
        norm = opt.clip_grad_norm(1.0)
        assert float(norm) == 6.0
        assert torch.equal(param.grad.cpu(), expect if mode == "eager" else unclipped), mode
        assert (param.grad._version > before) == (mode == "eager")
        if mode == "materialize":
            opt.materialize_pending()
            assert torch.equal(param.grad.cpu(), expect)
        version = param.grad._version
        opt.step()
        if mode == "defer":
            assert torch.equal(param.grad.cpu(), unclipped)
        else:
            assert torch.equal(param.grad.cpu(), expect)
            assert abs(float(param.grad.double().norm()) - 1.0) < 1e-5
            # the write-back is an in-place change: it bumps the version counter
            assert (param.grad._version > version) == (mode == "write_back")
        results[mode] = param.detach().cpu()
    for mode in ("write_back", "materialize", "defer"):
        assert torch.equal(results["eager"], results[mode]), mode


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_clip_then_read_grad_without_a_step(device, dtype):
    """The default clip leaves ``.grad`` clipped as soon as ``clip_grad_norm`` returns,
    with no step: a caller that logs or checks the clipped gradients, or hands them to a
    plain torch optimizer, reads the reference's values.  Several tensors (one of them
    misaligned and ragged) clipped by a multiplier that is not a power of two, compared
    bitwise with the oracle's ``grad.mul_``; a norm below the threshold leaves every bit,
    a bf16 NaN payload included, untouched (the reference multiplies only below 1).  The
    expected gradients are the reference's own op, ``grad.mul_(coefficient)`` with the
    Python-double coefficient, run by torch on the CPU."""
    gen = torch.Generator(device=device).manual_seed(31)
    sizes = (70_001, 4096, 33)
    grads = [(torch.randn(n + 1, device=device, generator=gen) * 0.37).to(dtype)[1:] for n in sizes]
    params = [torch.nn.Parameter(torch.zeros(g.shape, dtype=dtype, device=device)) for g in grads]
    for p, g in zip(params, grads):
        p.grad = g.clone()
    opt = ShardedOptimizer(params, OptimizerConfig(), norm_group=GroupHandle.trivial(), device=device)
    ints = torch.int32 if dtype == torch.float32 else torch.int16

    def host(t):
        t = t.detach().cpu()
        return t.numpy() if dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)

    ref_sq = sum(oracle.sqnorm(host(g)) for g in grads)
    norm = float(opt.clip_grad_norm(1.0))
    assert abs(norm**2 - ref_sq) <= 1e-12 * ref_sq
    coef = 1.0 / (norm + 1e-6)  # sharded_optimizer.py:331-337, a Python double
    assert coef < 1.0 and math.frexp(coef)[0] != 0.5
    for p, g in zip(params, grads):
        want = g.cpu().mul_(coef)
        assert torch.equal(p.grad.cpu().view(ints), want.view(ints))

    quiet = torch.zeros(9, dtype=dtype, device=device)
    quiet[3] = 1e-3
    if dtype == torch.bfloat16:
        quiet.view(torch.int16)[5] = 0x7FA1  # a NaN with a payload the store would not keep
    q = torch.nn.Parameter(torch.zeros(9, dtype=dtype, device=device))
    q.grad = quiet.clone()
    opt = ShardedOptimizer([q], OptimizerConfig(), norm_group=GroupHandle.trivial(), device=device)
    opt.clip_grad_norm(1e9 if dtype == torch.float32 else 1.0)
    assert torch.equal(q.grad.view(ints), quiet.view(ints))


def test_gradients_changed_after_the_clip(device):
    """The step applies the clip ``clip_grad_norm`` computed.  A gradient changed in place
    in between (its version counter moves) can no longer be clipped where the reference
    clipped it, so the step refuses rather than clipping the changed values; after
    ``materialize_pending`` (the reference's in-place clip, done at once) the same change
    is fine, and the result is the reference's clip-then-change sequence, bitwise."""
    from hybrid_training_amd.errors import ShardingError

    gen = torch.Generator(device=device).manual_seed(8)
    g0 = torch.randn(10_000, device=device, generator=gen)
    p0 = torch.randn(10_000, device=device, generator=gen) * 0.02
    param = torch.nn.Parameter(p0.clone())
    param.grad = g0.clone()
    opt = _make_optimizer([param], in_step=True)
    opt.clip_grad_norm(1.0)
    param.grad.mul_(0.5)  # changed after the clip
    with pytest.raises(ShardingError, match="materialize_pending"):
        opt.step()

    # the same sequence with the clip multiplier applied by hand, then the change
    ref = torch.nn.Parameter(p0.clone())
    ref_norm = None
    for mode in ("materialize", "eager"):
        param = torch.nn.Parameter(p0.clone())
        param.grad = g0.clone()
        opt = _make_optimizer([param], in_step=mode == "materialize")
        norm = float(opt.clip_grad_norm(1.0))
        if mode == "materialize":
            opt.materialize_pending()
        param.grad.mul_(0.5)
        opt.step()
        if ref_norm is None:
            ref_norm = norm
            ref.grad = (g0 * oracle.clip_multiplier(norm, 1.0)) * 0.5
            _make_optimizer([ref]).step()
        assert norm == ref_norm
        assert torch.equal(param.grad, ref.grad), mode
        assert torch.equal(param.detach(), ref.detach()), mode


def test_deferred_and_fused_paths_are_bitwise_equal(device):
    n = 300_007
    grads = [torch.randn(n, device=device) * 1e-2 for _ in range(3)]
    p0 = torch.randn(n, device=device) * 0.02
    results = []
    for mode in ("inplace", "defer", "fused"):
        param = torch.nn.Parameter(p0.clone())
        opt = _make_optimizer([param], defer=(mode == "defer"))
        for g in grads:
            param.grad = g.clone()
            if mode == "fused":
                norm = opt.clip_and_step(0.5)
            else:
                norm = opt.clip_grad_norm(0.5)
                opt.step()
            mul = oracle.clip_multiplier(float(norm), 0.5)
            clipped = (g.cpu() * np.float32(mul)) if mode != "defer" else g.cpu()
            assert torch.equal(param.grad.cpu(), clipped), mode
            opt.zero_grad()
        results.append(param.detach().clone())
    assert torch.equal(results[0], results[1]) and torch.equal(results[0], results[2])


def test_many_parameters_and_state_dict_round_trip(device):
    shapes = [(25, 14), (25,), (25, 25), (25,), (25, 25), (25,), (7, 25), (7,)] * 3
    params = [torch.nn.Parameter(torch.randn(s, device=device) * 0.1) for s in shapes]
    opt = _make_optimizer(params, lr=1e-3, betas=(0.9, 0.999), wd=0.01)
    expected = [p.detach().cpu().numpy().reshape(-1).copy() for p in params]
    ms = [np.zeros_like(e) for e in expected]
    vs = [np.zeros_like(e) for e in expected]
    for step in range(1, 4):
        for p in params:
            p.grad = torch.randn_like(p) * 1e-2
        grads = [p.grad.cpu().numpy().reshape(-1) for p in params]
        norm = float(opt.clip_grad_norm(0.05))
        mul = oracle.clip_multiplier(norm, 0.05)
        opt.step()
        sc = oracle.adamw_scalars(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
                                  step=float(step))
        for e, g, m, v in zip(expected, grads, ms, vs):
            oracle.adamw_step(e, g, m, v, sc, grad_mul=mul)
    for p, e in zip(params, expected):
        assert np.array_equal(p.detach().cpu().numpy().reshape(-1).view(np.int32), e.view(np.int32))
    saved = opt.state_dict()
    assert saved["num_parameters"] == len(params)
    fresh = _make_optimizer(params, lr=1e-3, betas=(0.9, 0.999), wd=0.01)
    fresh.load_state_dict(saved)
    assert float(fresh.inner.state[params[0]]["step"]) == 3.0
    assert fresh.state_bytes() == opt.state_bytes() == 2 * 4 * sum(p.numel() for p in params) + 4 * len(params)


def test_loaded_non_contiguous_state_steps_like_dense_state(device):
    """State tensors loaded with another layout (here transposed, non-contiguous) are
    placed dense, so the next step is bitwise the step from the saved dense state."""
    params = [torch.nn.Parameter(torch.randn(s, device=device) * 0.1) for s in [(33, 17), (17,), (8, 64)]]
    opt = _make_optimizer(params, lr=1e-3, betas=(0.9, 0.999), wd=0.01)
    for p in params:
        p.grad = torch.randn_like(p) * 1e-2
    opt.clip_grad_norm(1.0)
    opt.step()
    saved = opt.state_dict()
    # Separate copies: torch's load_state_dict keeps the loaded "step" tensor itself.
    strided = copy.deepcopy(saved)
    for entry in strided["state"].values():
        for k, v in entry.items():
            if torch.is_tensor(v) and v.dim() == 2:
                entry[k] = v.t().contiguous().t()
    assert any(not v.is_contiguous() for e in strided["state"].values() for v in e.values() if torch.is_tensor(v))
    copies = [torch.nn.Parameter(p.detach().clone()) for p in params]
    dense = _make_optimizer([torch.nn.Parameter(p.detach().clone()) for p in params], lr=1e-3,
                            betas=(0.9, 0.999), wd=0.01)
    dense_params = dense.parameters
    dense.load_state_dict(copy.deepcopy(saved))
    other = _make_optimizer(copies, lr=1e-3, betas=(0.9, 0.999), wd=0.01)
    other.load_state_dict(strided)
    for a, b in zip(dense_params, copies):
        a.grad = torch.ones_like(a) * 1e-3
        b.grad = torch.ones_like(b) * 1e-3
    for o in (dense, other):
        o.clip_grad_norm(1.0)
        o.step()
    for a, b in zip(dense_params, copies):
        assert torch.equal(a.detach().view(torch.int32), b.detach().view(torch.int32))


@pytest.mark.parametrize("name", ["adamw", "sgd"])
@pytest.mark.parametrize("offload", [False, True])
def test_refused_step_changes_no_state(device, name, offload):
    """A step refused for one parameter (a non-dense gradient, listed after a good one)
    creates no state and advances no step counter for any parameter: once the gradient
    is made dense, the step is bitwise a fresh optimizer's first step."""
    torch.manual_seed(5)
    shapes = [(300,), (17, 5)]
    init = [torch.randn(s) * 0.1 for s in shapes]
    grads = [torch.randn(s) * 1e-2 for s in shapes]
    config = OptimizerConfig(name=name, learning_rate=1e-2, weight_decay=0.01, momentum=0.9,
                             cpu_offload_state=offload)

    def make():
        params = [torch.nn.Parameter(t.to(device)) for t in init]
        return params, ShardedOptimizer(params, config, norm_group=GroupHandle.trivial(), device=device)

    params, opt = make()
    params[0].grad = grads[0].to(device)
    params[1].grad = grads[1].t().contiguous().to(device).t()  # the right shape, not dense
    with pytest.raises(ShardingError, match="dense"):
        opt.step()  # (the norm pass refuses the gradient before the update is reached)
    assert len(opt.inner.state) == 0
    assert torch.equal(params[0].detach().cpu(), init[0]) and torch.equal(params[1].detach().cpu(), init[1])
    params[1].grad = grads[1].to(device)
    opt.clip_grad_norm(1.0)
    opt.step()

    fresh, fresh_opt = make()
    for q, g in zip(fresh, grads):
        q.grad = g.to(device)
    fresh_opt.clip_grad_norm(1.0)
    fresh_opt.step()
    for a, b in zip(params, fresh):
        assert torch.equal(a.detach().view(torch.int32), b.detach().view(torch.int32))
        assert torch.equal(a.grad.view(torch.int32), b.grad.view(torch.int32))
    # (with state offload the state is keyed by the parameters' host copies)
    for a, b in zip(opt.inner.param_groups[0]["params"], fresh_opt.inner.param_groups[0]["params"]):
        assert fresh_opt.inner.state[b]
        for key, value in fresh_opt.inner.state[b].items():
            assert torch.equal(opt.inner.state[a][key].cpu(), value.cpu()), key


def test_norm_contributions_as_the_reference_tests_them(device):
    """``tests/unit/test_single_process_components.py:364-406`` on the device: the
    elementwise weights (2, 2, 1, 0) over 4 ranks on a ones gradient give 1.25; a
    parameter without a gradient contributes exactly 0; at world size 1 the norm of an
    MLP's gradients equals ``torch.nn.utils.clip_grad_norm_``'s (the reference's 1e-5
    bound: torch sums in fp32, this in fp64); a gradient of norm 6 clipped to 1 comes out
    at norm 1 once the clip lands in ``.grad`` (``materialize_pending``, or the step)."""
    from hybrid_training_amd import build_gradient_norm_contributions

    p = torch.nn.Parameter(torch.ones(4, device=device))
    p.grad = torch.ones(4, device=device)
    p.gradient_norm_scale_vector = torch.tensor([2.0, 2.0, 1.0, 0.0])
    assert build_gradient_norm_contributions([p], world_size=4)[0].squared_norm().item() == 1.25
    q = torch.nn.Parameter(torch.ones(4, device=device))
    assert build_gradient_norm_contributions([q], world_size=1)[0].squared_norm().item() == 0.0

    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(4, 8), torch.nn.ReLU(), torch.nn.Linear(8, 2)).to(device)
    model(torch.randn(3, 4, device=device)).sum().backward()
    expected = torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm=float("inf"))
    opt = ShardedOptimizer(list(model.parameters()), OptimizerConfig(), norm_group=GroupHandle.trivial(),
                           device=device)
    assert abs(opt.clip_grad_norm(0.0).item() - expected.item()) <= 1e-5

    r = torch.nn.Parameter(torch.ones(4, device=device))
    r.grad = torch.full((4,), 3.0, device=device)
    opt = ShardedOptimizer([r], OptimizerConfig(), norm_group=GroupHandle.trivial(), device=device)
    assert opt.clip_grad_norm(1.0).item() == pytest.approx(6.0)
    opt.materialize_pending()
    assert r.grad.norm().item() == pytest.approx(1.0, abs=1e-5)


def test_pending_unscale_is_read_through(device):
    n = 5000
    g = torch.randn(n, device=device) * 65536
    p0 = torch.randn(n, device=device)
    a = torch.nn.Parameter(p0.clone())
    b = torch.nn.Parameter(p0.clone())
    a.grad = g.clone()
    setattr(a.grad, PENDING_UNSCALE_ATTR, 2.0**-16)
    b.grad = g.clone().mul_(2.0**-16)
    for param in (a, b):
        opt = _make_optimizer([param])
        opt.clip_grad_norm(0.1)
        opt.step()
    assert torch.equal(a.detach(), b.detach())
    # in-place semantics: both gradients end unscaled and clipped, the factor consumed
    assert torch.equal(a.grad, b.grad) and not hasattr(a.grad, PENDING_UNSCALE_ATTR)


def test_full_size_llama_shard(device):
    n = LLAMA_SHARD
    gen = torch.Generator(device=device).manual_seed(0)
    param = torch.nn.Parameter(torch.randn(n, device=device, generator=gen) * 0.02)
    opt = _make_optimizer([param])
    idx = torch.randint(0, n, (1 << 20,), device=device, generator=gen)
    idx[0], idx[1] = 0, n - 1
    P = param.detach()[idx].cpu().numpy()
    M = np.zeros(idx.numel(), np.float32)
    V = np.zeros(idx.numel(), np.float32)
    for step in (1, 2):
        param.grad = torch.randn(n, device=device, generator=gen) * 1e-4
        G = param.grad[idx].cpu().numpy()
        ref = float(param.grad.double().pow(2).sum())
        norm = opt.clip_and_step(1.0)
        assert abs(float(norm) ** 2 - ref) <= 1e-10 * ref
        mul = oracle.clip_multiplier(float(norm), 1.0)
        assert mul < 1.0  # norm ~ sqrt(n) * 1e-4 ~ 3.17: clipping is active
        sc = oracle.adamw_scalars(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1,
                                  step=float(step))
        oracle.adamw_step(P, G, M, V, sc, grad_mul=mul)
        state = opt.inner.state[param]
        assert np.array_equal(param.detach()[idx].cpu().numpy().view(np.int32), P.view(np.int32))
        assert np.array_equal(state["exp_avg"][idx].cpu().numpy().view(np.int32), M.view(np.int32))
        assert np.array_equal(state["exp_avg_sq"][idx].cpu().numpy().view(np.int32), V.view(np.int32))
        opt.zero_grad()
    del opt, param
    torch.cuda.empty_cache()


def test_learning_rate_schedule_without_weight_decay(device):
    """``set_learning_rate`` between steps (a scheduler) with weight decay 0 (the
    reference's ``OptimizerConfig`` default): bitwise the oracle, and torch's CPU
    AdamW for m and v (p within the square-root tolerance)."""
    n = 50_001
    gen = torch.Generator(device=device).manual_seed(31)
    param = torch.nn.Parameter(torch.randn(n, device=device, generator=gen))
    opt = ShardedOptimizer([param], OptimizerConfig(learning_rate=1e-3, weight_decay=0.0),
                           norm_group=GroupHandle.trivial(), device=device)
    ref = torch.nn.Parameter(param.detach().cpu().clone())
    ref_opt = torch.optim.AdamW([ref], lr=1e-3, weight_decay=0.0, foreach=False)
    host_p = param.detach().cpu().numpy().copy()
    host_m = np.zeros(n, np.float32)
    host_v = np.zeros(n, np.float32)
    for step, lr in enumerate((1e-3, 7.5e-4, 5e-4, 2.5e-4), start=1):
        opt.set_learning_rate(lr)
        for group in ref_opt.param_groups:
            group["lr"] = lr
        g = torch.randn(n, device=device, generator=gen) * 1e-2
        param.grad = g
        ref.grad = g.cpu()
        opt.step()
        ref_opt.step()
        sc = oracle.adamw_scalars(lr=lr, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, step=float(step))
        oracle.adamw_step(host_p, g.cpu().numpy(), host_m, host_v, sc)
        got = param.detach().cpu().numpy()
        assert np.array_equal(got.view(np.int32), host_p.view(np.int32)), step
        state = opt.inner.state[param]
        assert torch.equal(state["exp_avg"].cpu(), ref_opt.state[ref]["exp_avg"])
        assert torch.equal(state["exp_avg_sq"].cpu(), ref_opt.state[ref]["exp_avg_sq"])
        rel = np.abs(got - ref.detach().numpy()) / np.maximum(np.abs(ref.detach().numpy()), lr)
        assert float(rel.max()) <= 1e-6
    assert opt.learning_rate == 2.5e-4
