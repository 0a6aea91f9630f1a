"""The reference's CPU op sequences on the hot path (CPU baselines only).

TEST/BENCH INFRASTRUCTURE ONLY: ``bench.py`` times these as its CPU baselines.

:class:`ReferenceCpuStep` restates, with the same torch CPU ops, what the reference runs
per step on a flat shard: ``NormContribution.squared_norm``
(``optim/sharded_optimizer.py:151-158``: ``grad.to(float64).pow(2)`` then ``sum``),
``distributed_gradient_norm``'s ``clamp_min(0).sqrt()`` (``:241``), the clip
(``:333-337``: ``.item()``, Python-double coefficient, ``grad.mul_``) and the inner
optimizer's ``step`` (``:355``): ``torch.optim.AdamW`` (``torch/optim/adam.py:347-547``)
or ``torch.optim.SGD`` (``torch/optim/sgd.py``), the single-tensor paths on CPU tensors.
The functions below restate the reference's other op sequences on the path: the DDP
bucket pack, the FSDP shard build, gather and unpack, the reduce-scatter's AVG
arithmetic on one rank's share (plain and at the end of a ``no_sync`` accumulation), the
checkpoint re-slice and the loss scaler's unscale and finiteness check.
"""

from __future__ import annotations

import math

import torch


class ReferenceCpuStep:
    """One flat shard (fp32 unless ``dtype`` says otherwise: the parameters' own dtype
    with mixed precision off) with its gradient and a torch CPU AdamW or SGD."""

    def __init__(self, numel: int, *, lr: float, betas: tuple[float, float], eps: float,
                 weight_decay: float, seed: int = 0, momentum: float | None = None,
                 dtype: torch.dtype = torch.float32) -> None:
        gen = torch.Generator().manual_seed(seed)
        self.param = torch.nn.Parameter((torch.randn(numel, generator=gen) * 0.02).to(dtype))
        self.grad = (torch.randn(numel, generator=gen) * 1e-4).to(dtype)
        if momentum is None:
            self.optimizer = torch.optim.AdamW(
                [self.param], lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, foreach=False
            )
        else:  # optim/sharded_optimizer.py:121-126
            self.optimizer = torch.optim.SGD([self.param], lr=lr, momentum=momentum, weight_decay=weight_decay,
                                             foreach=False)

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


def pack_buckets(buckets: list[tuple[torch.Tensor, list[tuple[int, torch.Tensor]]]], world: int) -> None:
    """The DDP bucket pack: each gradient copied into its bucket slice
    (``parallel/ddp.py:513``, ``bucket.view_for(position).copy_(param.grad)``), then each
    bucket divided by the group size before its all-reduce
    (``distributed/collectives.py:366-367``, ``tensor.div_(group.size)``).
    ``buckets``: (bucket buffer, [(offset, gradient), ...]) in launch order."""
    for buffer, members in buckets:
        for offset, grad in members:
            buffer[offset : offset + grad.numel()].copy_(grad.reshape(-1))
        buffer.div_(world)


def build_shard(params: list[torch.Tensor], padded_numel: int, shard_numel: int, rank: int,
                master_dtype: torch.dtype) -> torch.Tensor:
    """``FlatParamHandle._build_shard`` (``parallel/fsdp.py:433-454``): a zero padded flat
    buffer in the master dtype, every parameter copied in at its offset (cast), and this
    rank's slice cloned."""
    flat = torch.zeros(padded_numel, dtype=master_dtype)
    offset = 0
    for p in params:
        flat[offset : offset + p.numel()].copy_(p.detach().to(dtype=master_dtype).reshape(-1))
        offset += p.numel()
    start = rank * shard_numel
    shard = flat[start : start + shard_numel].clone()
    del flat
    return shard


def gather_full(shards: list[torch.Tensor], compute_dtype: torch.dtype) -> torch.Tensor:
    """``FlatParamHandle.gather_full`` (``parallel/fsdp.py:564-591``) for every rank's shard:
    each shard cast to the compute dtype, then the all-gather placing each cast shard in
    the full padded buffer."""
    size = shards[0].numel()
    full = torch.empty(size * len(shards), dtype=compute_dtype)
    for q, shard in enumerate(shards):
        full[q * size : (q + 1) * size].copy_(shard.to(compute_dtype))
    return full


def full_tensors(shards: list[torch.Tensor], entries: list[tuple[int, tuple[int, ...]]]) -> list[torch.Tensor]:
    """``FlatParamHandle.full_tensors`` (``parallel/fsdp.py:912-925``): the all-gathered
    flat buffer, then every parameter cloned out of it as a shaped view.
    ``entries``: (offset, shape) per parameter."""
    full = torch.cat(shards)
    return [full[offset : offset + math.prod(shape)].view(shape).clone() for offset, shape in entries]


def local_share(grads: list[torch.Tensor], rows: list[torch.Tensor] | None, world: int,
                reduce_dtype: torch.dtype, master_dtype: torch.dtype) -> torch.Tensor:
    """The AVG reduce-scatter's arithmetic on one rank's share: each rank's slice cast to
    the reduce dtype (``parallel/fsdp.py:734-735``) and divided by the group size
    (``distributed/collectives.py:593-594``, ``tensor.div(group.size)``), the slices summed
    in rank order (the collective's sum), the result cast to the master dtype
    (``parallel/fsdp.py:760-761``).  With ``rows`` (the end of a ``no_sync``
    accumulation, ``parallel/fsdp.py:747-749``) each slice is first added to its
    accumulated row (``grad + accumulator``)."""
    out = None
    for q, g in enumerate(grads):
        x = g.to(reduce_dtype)
        if rows is not None:
            x = x + rows[q]
        part = x.div(world)
        out = part if out is None else out.add_(part)
    return out.to(master_dtype)


def read_pieces_into_shard(shard: torch.Tensor, pieces: list[tuple[int, list[torch.Tensor]]]) -> None:
    """The checkpoint re-slice into one destination flat shard: per owned piece,
    ``read_tensor_range`` fills a fresh tensor from every intersecting stored interval
    (``checkpoint/reshard.py:286-290``, ``out[filled : filled + n] = flat[...].to(out.dtype)``)
    and the piece is copied into the shard at its local offset (``parallel/fsdp.py:862-910``).
    ``pieces``: (local offset, [stored intervals in order]) per owned piece."""
    for local_offset, intervals in pieces:
        length = sum(int(t.numel()) for t in intervals)
        out = torch.empty(length, dtype=shard.dtype)
        filled = 0
        for stored in intervals:
            out[filled : filled + stored.numel()] = stored.to(out.dtype)
            filled += stored.numel()
        shard[local_offset : local_offset + length].copy_(out)


def unscale_and_check(grads: list[torch.Tensor], scale: float) -> bool:
    """``GradScaler.unscale_`` (``optim/grad_scaler.py:181-186``: ``grad.mul_(1 / scale)``)
    and ``_detect_non_finite``'s scan (``:191-199``: ``torch.isfinite(grad).all()`` per
    gradient until the first non-finite one)."""
    inverse = 1.0 / scale
    for g in grads:
        g.mul_(inverse)
    for g in grads:
        if not bool(torch.isfinite(g).all()):
            return True
    return False


class ReferenceMlpTail:
    """The per-step tail of the reference's FSDP MLP training at group size ``world``, all
    ranks on this host (``tests/distributed/test_fsdp.py:86-151`` trains it with Gloo):
    each rank's share of the AVG reduce-scatter of the ranks' padded flat gradients
    (:func:`local_share`), the global gradient norm (each rank's ``grad.to(float64)
    .pow(2).sum()``, the all-reduce's sum in rank order, ``clamp_min(0).sqrt()``,
    ``optim/sharded_optimizer.py:151-158, 241``), the clip (``:333-337``) and each rank's
    ``torch.optim.AdamW`` step on its flat shard (``:355``)."""

    def __init__(self, full_grads: list[torch.Tensor], shard: int, *, lr: float, weight_decay: float,
                 seed: int = 0) -> None:
        gen = torch.Generator().manual_seed(seed)
        self.world = len(full_grads)
        self.shard = shard
        self.grads = [g.detach().cpu().float().reshape(-1) for g in full_grads]
        self.params = [torch.nn.Parameter(torch.randn(shard, generator=gen) * 0.1) for _ in range(self.world)]
        self.optimizers = [torch.optim.AdamW([p], lr=lr, weight_decay=weight_decay, foreach=False)
                           for p in self.params]

    def step(self, max_norm: float) -> float:
        """One step of every rank; returns the pre-clip global norm."""
        shares = []
        for rank in range(self.world):
            lo = rank * self.shard
            shares.append(local_share([g[lo : lo + self.shard] for g in self.grads], None, self.world,
                                      torch.float32, torch.float32))
        squared = None
        for share in shares:
            part = share.to(torch.float64).pow(2).sum()
            squared = part if squared is None else squared + part
        norm = float(squared.clamp_min(0).sqrt())
        coefficient = float(max_norm) / (norm + 1e-6)
        for p, share, opt in zip(self.params, shares, self.optimizers):
            if coefficient < 1.0:
                share.mul_(coefficient)
            p.grad = share
            opt.step()
            p.grad = None
        return norm
