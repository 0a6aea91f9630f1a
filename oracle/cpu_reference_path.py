"""The reference's CPU op sequence for one clipped AdamW step (CPU baseline only).

TEST/BENCH INFRASTRUCTURE ONLY: ``bench.py`` times this as the CPU baseline.

It restates, with the same torch CPU ops, what the reference runs per step on a
flat shard: ``NormContribution.squared_norm`` (``optim/sharded_optimizer.py:151-158``:
``grad.to(float64).pow(2)`` then ``sum``), ``distributed_gradient_norm``'s
``clamp_min(0).sqrt()`` (``:241``), the clip (``:333-337``: ``.item()``, Python-double
coefficient, ``grad.mul_``) and ``torch.optim.AdamW.step`` (``:355`` ->
``torch/optim/adam.py:347-547``, the single-tensor path on CPU tensors).
"""

from __future__ import annotations

import torch


class ReferenceCpuStep:
    """One flat fp32 shard with its gradient and a torch CPU AdamW."""

    def __init__(self, numel: int, *, lr: float, betas: tuple[float, float], eps: float,
                 weight_decay: float, seed: int = 0) -> None:
        gen = torch.Generator().manual_seed(seed)
        self.param = torch.nn.Parameter(torch.randn(numel, generator=gen) * 0.02)
        self.grad = torch.randn(numel, generator=gen) * 1e-4
        self.optimizer = torch.optim.AdamW(
            [self.param], lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, foreach=False
        )

    def prepare(self) -> None:
        """Attach a fresh gradient (stands in for backward; not part of the timed step)."""
        self.param.grad = self.grad.clone()

    def step(self, max_norm: float) -> float:
        """Norm, clip and update; returns the pre-clip norm."""
        squared = self.param.grad.detach().to(torch.float64).pow(2).sum()
        norm = squared.reshape(1)[0].clamp_min(0).sqrt()
        coefficient = float(max_norm) / (float(norm.item()) + 1e-6)
        if coefficient < 1.0:
            self.param.grad.detach().mul_(coefficient)
        self.optimizer.step()
        self.param.grad = None
        return float(norm)
