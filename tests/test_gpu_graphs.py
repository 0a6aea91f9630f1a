"""StepGraph: the drop-in tail recorded once into a HIP graph and replayed.

Two copies of the same FSDP setup (the reference's 1,857-parameter MLP as W ranks'
flat units, each with its ShardedOptimizer) take the same steps: one eagerly, one by
replaying a recording of its first copy's step function.  Between steps the program
writes new gradients into the gradient buffers (eager device work between replays) and,
once, changes the learning rate.  After every step the parameters, gradients, optimizer
state, step counters and returned norms must be bitwise equal: a replay is the eager
step, with the step scalars (AdamW's bias corrections, the learning rate) taken from the
host state of that step.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
import torch.nn as nn

from hybrid_training_amd import (
    BucketedGradients,
    DDPConfig,
    FlatParamHandle,
    FSDPConfig,
    GroupHandle,
    MixedPrecisionConfig,
    OptimizerConfig,
    ShardedOptimizer,
    StepGraph,
    UnsupportedFeatureError,
)
from hybrid_training_amd import _native
from hybrid_training_amd.optim import PENDING_UNSCALE_ATTR

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
TOTAL = 1857


class _Tail:
    """W ranks' FSDP units of one MLP, their optimizers, and full gradients in fixed buffers."""

    def __init__(self, world: int, config: OptimizerConfig, dtype: torch.dtype = torch.float32,
                 mp: MixedPrecisionConfig | None = None, **placement):
        torch.manual_seed(0)
        model = nn.Sequential(nn.Linear(23, 32), nn.ReLU(), nn.Linear(32, 32), nn.ReLU(), nn.Linear(32, 1))
        named = list(model.to(DEV, dtype).named_parameters())
        mp = mp or MixedPrecisionConfig(enabled=False)
        self.handles = [FlatParamHandle(named, None, GroupHandle.local_view("shard", world, r), FSDPConfig(),
                                        mp, DEV, keep_originals=True)
                        for r in range(world)]
        padded = self.handles[0].padded_numel
        grad_dtype = getattr(torch, mp.param_dtype) if mp.enabled else dtype
        self.grads = [torch.zeros(padded, device=DEV, dtype=grad_dtype) for _ in range(world)]
        self.opts = [ShardedOptimizer([h.flat_param], config, norm_group=GroupHandle.local_view("world", world, r),
                                      device=DEV, **placement) for r, h in enumerate(self.handles)]

    def load_grads(self, k: int) -> None:
        gen = torch.Generator(device=DEV).manual_seed(100 + k)
        for g in self.grads:
            g.copy_(torch.randn(g.shape, device=DEV, generator=gen, dtype=torch.float32).to(g.dtype))
            g[TOTAL:] = 0.0  # the padding carries no gradient

    def step(self) -> list[torch.Tensor]:
        norms = []
        for r, (h, opt) in enumerate(zip(self.handles, self.opts)):
            h.flat_param.grad = h.reduce_scatter_gradient(self.grads[r], peer_grads=self.grads)
            norms.append(opt.clip_grad_norm(1.0))
            opt.step()
        return norms


def _assert_same(eager: _Tail, graphed: _Tail, eager_norms, graphed_norms, k: int) -> None:
    for r, (he, hg) in enumerate(zip(eager.handles, graphed.handles)):
        assert torch.equal(he.flat_param, hg.flat_param), (k, r, "param")
        assert torch.equal(he.flat_param.grad, hg.flat_param.grad), (k, r, "grad")
    for oe, og in zip(eager.opts, graphed.opts):
        (pe,), (pg,) = oe.parameters, og.parameters
        se, sg = oe.inner.state[pe], og.inner.state[pg]
        assert se.keys() == sg.keys()
        for key in se:
            assert torch.equal(se[key], sg[key]), (k, key)
    for ne, ng in zip(eager_norms, graphed_norms):
        assert torch.equal(ne, ng), (k, "norm")


def _run(world: int, config: OptimizerConfig, dtype=torch.float32, replays: int = 5, **placement) -> StepGraph:
    eager, graphed = _Tail(world, config, dtype, **placement), _Tail(world, config, dtype, **placement)
    for tail in (eager, graphed):
        tail.load_grads(0)
        tail.step()  # the eager step that creates the optimizer state
    graph = StepGraph(graphed.step)
    assert graph.recorded_steps == world
    for k in range(1, replays + 1):
        if k == 3:
            for tail in (eager, graphed):
                for opt in tail.opts:
                    opt.set_learning_rate(4e-4)
        for tail in (eager, graphed):
            tail.load_grads(k)
        norms = eager.step()
        graph.replay()
        torch.cuda.synchronize()
        _assert_same(eager, graphed, norms, graph.output, k)
    return graph


@pytest.mark.parametrize("world", [2, 4])
@pytest.mark.parametrize("placement", [{}, {"clip_in_step": True}, {"defer_clip": True}],
                         ids=["in_place_clip", "clip_in_step", "defer_clip"])
def test_recorded_adamw_tail_replays_the_eager_steps(world, placement):
    _run(world, OptimizerConfig(learning_rate=1e-3, weight_decay=0.01), **placement)


def test_recorded_sgd_tail_replays_the_eager_steps():
    _run(2, OptimizerConfig(name="sgd", learning_rate=1e-2, weight_decay=0.01, momentum=0.9))


@pytest.mark.parametrize("dtype", [torch.float64, torch.bfloat16], ids=["float64", "bfloat16"])
def test_recorded_tail_on_other_master_dtypes(dtype):
    _run(2, OptimizerConfig(learning_rate=1e-3, weight_decay=0.01), dtype, replays=3)
    _run(2, OptimizerConfig(name="sgd", learning_rate=1e-2, momentum=0.9), dtype, replays=3)


# A refused recording ends its capture early, sometimes before any launch.
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_recording_refuses_what_a_replay_cannot_repeat():
    config = OptimizerConfig(learning_rate=1e-3)
    tail = _Tail(2, config)
    tail.load_grads(0)
    # before any eager step the optimizer state does not exist yet
    with pytest.raises(UnsupportedFeatureError, match="creates the optimizer state"):
        StepGraph(tail.step)
    tail.step()
    # a pending loss-scale factor: the scaler decides on the host whether to skip
    grad = tail.handles[0].flat_param.grad
    setattr(grad, PENDING_UNSCALE_ATTR, 0.5)
    with pytest.raises(UnsupportedFeatureError, match="loss-scaled"):
        StepGraph(lambda: tail.opts[0].step())
    delattr(grad, PENDING_UNSCALE_ATTR)
    # a bare torch.cuda.graph capture of a step: its replays would keep the recorded scalars
    with pytest.raises(UnsupportedFeatureError, match="StepGraph"):
        with torch.cuda.graph(torch.cuda.CUDAGraph()):
            tail.opts[0].step()
    # a function that steps one optimizer twice
    with pytest.raises(UnsupportedFeatureError, match="twice"):
        StepGraph(lambda: (tail.opts[0].step(), tail.opts[0].step()))
    # the eager path still works after the refusals
    tail.step()
    torch.cuda.synchronize()


def test_replay_refuses_a_rebound_gradient_and_changes_nothing():
    tail = _Tail(2, OptimizerConfig(learning_rate=1e-3))
    tail.load_grads(0)
    tail.step()
    graph = StepGraph(tail.step)
    graph.replay()
    torch.cuda.synchronize()
    p = tail.handles[0].flat_param
    step_before = float(tail.opts[0].inner.state[p]["step"])
    kept = p.grad
    p.grad = kept.clone()
    with pytest.raises(UnsupportedFeatureError, match="rebound"):
        graph.replay()
    assert float(tail.opts[0].inner.state[p]["step"]) == step_before
    assert float(tail.opts[1].inner.state[tail.handles[1].flat_param]["step"]) == step_before
    p.grad = kept
    graph.replay()
    torch.cuda.synchronize()
    assert float(tail.opts[0].inner.state[p]["step"]) == step_before + 1


@pytest.mark.parametrize("config", [OptimizerConfig(learning_rate=1e-3),
                                    OptimizerConfig(name="sgd", learning_rate=1e-2, momentum=0.9)],
                         ids=["adamw", "sgd"])
def test_replay_refuses_replaced_parameters_or_state_and_changes_nothing(config):
    """load_state_dict places the optimizer state in new tensors, and an assignment to
    .data gives a parameter new storage: a replay would update the recorded tensors, so it
    refuses before changing anything, and a new recording replays again."""
    tail = _Tail(2, config)
    tail.load_grads(0)
    tail.step()
    graph = StepGraph(tail.step)
    graph.replay()
    torch.cuda.synchronize()
    opt = tail.opts[0]
    (p,) = opt.parameters
    state_before = {k: v.clone() for k, v in opt.inner.state[p].items()}
    params_before = [h.flat_param.detach().clone() for h in tail.handles]
    opt.load_state_dict(opt.state_dict())
    with pytest.raises(UnsupportedFeatureError, match="no longer the tensor"):
        graph.replay()
    torch.cuda.synchronize()
    for k, v in opt.inner.state[p].items():
        assert torch.equal(v, state_before[k]), k
    for h, before in zip(tail.handles, params_before):
        assert torch.equal(h.flat_param, before)
    if "step" in state_before:
        assert float(tail.opts[1].inner.state[tail.handles[1].flat_param]["step"]) == float(state_before["step"])
    graph = StepGraph(tail.step)  # recorded over the loaded state
    graph.replay()
    torch.cuda.synchronize()
    assert not torch.equal(tail.handles[0].flat_param, params_before[0])
    # what the eager step would do differently: a pending loss-scale factor, amsgrad
    # switched on, a parameter dropped from the optimizer
    grad = p.grad
    setattr(grad, PENDING_UNSCALE_ATTR, 0.5)
    with pytest.raises(UnsupportedFeatureError, match="loss-scale factor is pending"):
        graph.replay()
    delattr(grad, PENDING_UNSCALE_ATTR)
    group = opt.inner.param_groups[0]
    if "amsgrad" in group:
        group["amsgrad"] = True
        with pytest.raises(UnsupportedFeatureError, match="amsgrad or maximize"):
            graph.replay()
        group["amsgrad"] = False
    kept, group["params"] = group["params"], []
    with pytest.raises(UnsupportedFeatureError, match="no longer in the optimizer"):
        graph.replay()
    group["params"] = kept
    graph.replay()
    torch.cuda.synchronize()
    p.data = p.data.clone()
    with pytest.raises(UnsupportedFeatureError, match="no longer the tensor"):
        graph.replay()


@pytest.mark.parametrize("world", [2, 4])
def test_recorded_fsdp_step_with_the_parameter_gather(world):
    """The gather of every rank's fp32 master shard into the bf16 compute buffer (a cast
    copy of W records, whose interval table the recording writes into the graph) recorded
    with the tail: each replay's gathered buffers, shards and state bitwise the eager
    step's."""
    mp = MixedPrecisionConfig(enabled=True, param_dtype="bfloat16", reduce_dtype="float32", master_dtype="float32")
    config = OptimizerConfig(learning_rate=1e-3, weight_decay=0.01)
    eager, graphed = _Tail(world, config, mp=mp), _Tail(world, config, mp=mp)

    def step(tail: _Tail):
        shards = [h.flat_param for h in tail.handles]
        fulls = [h.gather_full(peer_shards=shards) for h in tail.handles]
        return fulls, tail.step()

    for tail in (eager, graphed):
        tail.load_grads(0)
        step(tail)
    graph = StepGraph(lambda: step(graphed))
    for k in range(1, 5):
        for tail in (eager, graphed):
            tail.load_grads(k)
        fulls, norms = step(eager)
        graph.replay()
        torch.cuda.synchronize()
        for fe, fg in zip(fulls, graph.output[0]):
            assert torch.equal(fe, fg), (k, "gathered")
        _assert_same(eager, graphed, norms, graph.output[1], k)


class _DdpTail:
    """One data-parallel replica: the MLP's parameters in several gradient buckets
    (gradient-as-bucket-view after the first synchronize) and one AdamW over them."""

    def __init__(self, world: int):
        torch.manual_seed(0)
        model = nn.Sequential(nn.Linear(23, 32), nn.ReLU(), nn.Linear(32, 32), nn.ReLU(), nn.Linear(32, 1))
        named = list(model.to(DEV).named_parameters())
        self.params = [p for _, p in named]
        group = GroupHandle.local_view("data_parallel", world, 0) if world > 1 else GroupHandle.trivial()
        # a 2 KiB cap puts the 1,857 parameters in several buckets
        self.ddp = BucketedGradients(named, group, DDPConfig(bucket_cap_mb=2.0 / 1024))
        self.opt = ShardedOptimizer(self.params, OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                                    norm_group=GroupHandle.trivial(), device=DEV)

    def load_grads(self, k: int) -> None:
        """New gradients in place, as a backward pass accumulating into zeroed
        gradients writes them (into the bucket views once they are bound)."""
        gen = torch.Generator(device=DEV).manual_seed(200 + k)
        for p in self.params:
            g = torch.randn(p.shape, device=DEV, generator=gen)
            if p.grad is None:
                p.grad = g
            else:
                p.grad.copy_(g)

    def step(self) -> torch.Tensor:
        self.ddp.synchronize()
        norm = self.opt.clip_grad_norm(1.0)
        self.opt.step()
        return norm


@pytest.mark.parametrize("world", [1, 2, 3])
def test_recorded_ddp_step_replays_the_eager_steps(world):
    """The data-parallel tail recorded: the bucket pack with its AVG divide by the group
    size (in place, the gradients being bucket views), the clip over every bucket view
    and AdamW; each replay bitwise the eager step, buckets included."""
    eager, graphed = _DdpTail(world), _DdpTail(world)
    assert len(graphed.ddp._buckets) > 2
    for tail in (eager, graphed):
        tail.load_grads(0)
        tail.step()  # packs the separate gradients, binds the views, creates the state
    graph = StepGraph(graphed.step)
    assert graph.recorded_steps == 1  # one launch group: every parameter shares its scalars
    for k in range(1, 6):
        if k == 3:
            for tail in (eager, graphed):
                tail.opt.set_learning_rate(4e-4)
        for tail in (eager, graphed):
            tail.load_grads(k)
        norm = eager.step()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(norm, graph.output), (k, "norm")
        for be, bg in zip(eager.ddp._buckets, graphed.ddp._buckets):
            assert torch.equal(be.buffer, bg.buffer), (k, "bucket")
        for pe, pg in zip(eager.params, graphed.params):
            assert torch.equal(pe, pg), (k, "param")
            se, sg = eager.opt.inner.state[pe], graphed.opt.inner.state[pg]
            for key in se:
                assert torch.equal(se[key], sg[key]), (k, key)


def test_recorded_training_step_with_forward_and_backward():
    """A whole data-parallel training step in one graph: torch's forward and backward
    (accumulating into the bound bucket views), the pack with its AVG divide, the clip
    and AdamW.  Between replays the program writes the next batch into the static
    input.  torch's matrix products may pick other kernels under capture than eagerly,
    so the comparison with the eager steps allows 1e-5 relative; the bucket pack and
    the optimizer alone replay bitwise (the tests above)."""
    eager, graphed = _ModelTail(), _ModelTail()
    x = torch.empty(64, 23, device=DEV)
    y = torch.empty(64, 1, device=DEV)

    def load_batch(k: int) -> None:
        gen = torch.Generator(device=DEV).manual_seed(300 + k)
        x.copy_(torch.randn(x.shape, device=DEV, generator=gen))
        y.copy_(torch.randn(y.shape, device=DEV, generator=gen))

    def step(tail: "_ModelTail") -> torch.Tensor:
        tail.opt.zero_grad(set_to_none=False)
        loss = nn.functional.mse_loss(tail.model(x), y)
        loss.backward()
        tail.ddp.synchronize()
        tail.opt.clip_grad_norm(1.0)
        tail.opt.step()
        return loss.detach()

    for tail in (eager, graphed):
        load_batch(0)
        for p in tail.model.parameters():
            p.grad = torch.zeros_like(p)
        step(tail)  # binds the bucket views and creates the optimizer state
    graph = StepGraph(lambda: step(graphed))
    start = [p.detach().clone() for p in graphed.model.parameters()]
    for k in range(1, 6):
        load_batch(k)
        loss = step(eager)
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(graph.output, loss, rtol=1e-5, atol=1e-7)
        for pe, pg in zip(eager.model.parameters(), graphed.model.parameters()):
            torch.testing.assert_close(pg, pe, rtol=1e-5, atol=1e-7)
            torch.testing.assert_close(pg.grad, pe.grad, rtol=1e-5, atol=1e-7)
    assert all(not torch.equal(s, p) for s, p in zip(start, graphed.model.parameters()))


class _ModelTail:
    """The MLP's parameters in 2 KiB gradient buckets (AVG over 2 replicas) with AdamW."""

    def __init__(self):
        torch.manual_seed(0)
        self.model = nn.Sequential(nn.Linear(23, 32), nn.ReLU(), nn.Linear(32, 32), nn.ReLU(),
                                   nn.Linear(32, 1)).to(DEV)
        named = list(self.model.named_parameters())
        self.ddp = BucketedGradients(named, GroupHandle.local_view("data_parallel", 2, 0),
                                     DDPConfig(bucket_cap_mb=2.0 / 1024))
        self.opt = ShardedOptimizer([p for _, p in named], OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                                    norm_group=GroupHandle.trivial(), device=DEV)


def test_slots_written_from_host_records_equal_the_writers():
    """Before a replay every recorded step's scalars are formatted on the host
    (hbt_*_scalar_record) and all slots are written by one hbt_write_words call: the
    slots must be bitwise what each step's own writer (hbt_*_write_scalars) leaves, for
    every kind of step, with zeros after each record."""
    lib = _native.library()
    size = _native.STEP_SLOT_BYTES
    rng = np.random.default_rng(11)
    slots = 13  # two launches of at most 8 slots (256 words)
    by_writers = torch.zeros(slots * size // 8, dtype=torch.float64, device=DEV)
    together = torch.full_like(by_writers, float("nan"))
    records = (ctypes.c_uint8 * (slots * size))()
    stream = _native.stream_of(DEV)
    momentum = int(_native.SGD_MOMENTUM)
    for i in range(slots):
        slot = by_writers.data_ptr() + i * size
        record = ctypes.addressof(records) + i * size
        values = [float(v) for v in rng.uniform(-2.0, 2.0, 7)]
        dtype = int(i % 3)  # F32, BF16, F16
        unscale = float(rng.choice([1.0, 2.0**-16]))
        kind = i % 4
        if kind == 0:
            assert lib.hbt_adamw_write_scalars(slot, dtype, unscale, *values, stream) == 0
            assert lib.hbt_adamw_scalar_record(record, dtype, unscale, *values) == 0
        elif kind == 1:
            assert lib.hbt_adamw_write_scalars_f64(slot, unscale, *values, stream) == 0
            assert lib.hbt_adamw_scalar_record_f64(record, unscale, *values) == 0
        elif kind == 2:
            assert lib.hbt_sgd_write_scalars(slot, dtype, unscale, *values[:4], momentum, stream) == 0
            assert lib.hbt_sgd_scalar_record(record, dtype, unscale, *values[:4], momentum) == 0
        else:
            assert lib.hbt_sgd_write_scalars_f64(slot, unscale, *values[:4], 0, stream) == 0
            assert lib.hbt_sgd_scalar_record_f64(record, unscale, *values[:4], 0) == 0
    words = ctypes.cast(records, ctypes.POINTER(ctypes.c_uint32))
    assert lib.hbt_write_words(together.data_ptr(), words, slots * size // 4, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(by_writers.view(torch.int32), together.view(torch.int32))


@pytest.mark.parametrize("count", [1, 63, 64, 65, 255, 256, 257, 700])
def test_write_words_across_blocks_and_launches(count):
    """hbt_write_words carries up to 256 words per launch, 64 per block: every word lands
    at its index and nothing past the count is touched."""
    lib = _native.library()
    rng = np.random.default_rng(count)
    words = rng.integers(0, 2**32, count, dtype=np.uint64).astype(np.uint32)
    dst = torch.full((count + 70,), -1, dtype=torch.int32, device=DEV)
    host = (ctypes.c_uint32 * count)(*[int(w) for w in words])
    assert lib.hbt_write_words(dst.data_ptr(), host, count, _native.stream_of(DEV)) == 0
    torch.cuda.synchronize()
    got = dst.cpu().numpy().view(np.uint32)
    assert np.array_equal(got[:count], words)
    assert np.all(got[count:] == np.uint32(0xFFFFFFFF))


@pytest.mark.parametrize("world", [2, 4])
def test_recorded_no_sync_cycle(world):
    """A whole gradient-accumulation cycle recorded: one micro-batch accumulated without
    reduction (no_sync), the next added to it and reduced in one pass, then the clip and
    AdamW.  The accumulator rows the first micro-batch allocates belong to the graph, and
    each replay repeats the cycle from its first micro-batch; every replay is bitwise the
    eager cycle."""
    config = OptimizerConfig(learning_rate=1e-3, weight_decay=0.01)
    eager, graphed = _Tail(world, config), _Tail(world, config)
    micro = [[torch.empty_like(g) for g in eager.grads] for _ in range(2)]

    def load(k: int) -> None:
        gen = torch.Generator(device=DEV).manual_seed(700 + k)
        for batch in micro:
            for g in batch:
                g.copy_(torch.randn(g.shape, device=DEV, generator=gen))
                g[TOTAL:] = 0.0

    def cycle(tail: _Tail) -> list[torch.Tensor]:
        norms = []
        for r, (h, opt) in enumerate(zip(tail.handles, tail.opts)):
            h.set_accumulate_without_reduction(True)
            assert h.reduce_scatter_gradient(micro[0][r], peer_grads=micro[0]) is None
            h.set_accumulate_without_reduction(False)
            h.flat_param.grad = h.reduce_scatter_gradient(micro[1][r], peer_grads=micro[1])
            norms.append(opt.clip_grad_norm(1.0))
            opt.step()
        return norms

    load(0)
    for tail in (eager, graphed):
        cycle(tail)
    graph = StepGraph(lambda: cycle(graphed))
    assert not any(h.has_pending_accumulation for h in graphed.handles)
    for k in range(1, 5):
        load(k)
        norms = cycle(eager)
        graph.replay()
        torch.cuda.synchronize()
        _assert_same(eager, graphed, norms, graph.output, k)
