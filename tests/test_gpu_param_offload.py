"""GPU parity of parameter CPU offload (``FSDPConfig.cpu_offload_params``).

Reference behaviour: the persistent shard lives on the host (``parallel/fsdp.py:450-451``),
is copied to the device for every gather (``:575-577``, ``:690-691``) and unpack
(``:919``), the reduce-scattered gradient shard is moved to the host (``:763-764``),
and the optimizer steps the host shard where it lies.  The reference's own test
(``tests/unit/test_single_process_components.py:300-345``) asserts that offload changes
neither the gradient nor the update.  Here every pass over a host tensor streams it
through the device, so each check is that the bits equal those of the same values in
HBM:

* the handle: shard, gather, unpack, gradient shard and its norm partials, pieces and a
  checkpoint round trip;
* the optimizer on host-resident parameters: norm, clip and AdamW / SGD steps with
  random sizes, chunkings, master dtypes and clip placement (parameters, gradients and
  state), and for fp32 the oracle;
* the norm pass over host gradients at every 16-byte alignment;
* the loss scaler's eager unscale and overflow check on host gradients;
* ``no_sync`` accumulation and the gathered buffer's storage cycle on an offloaded unit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from hybrid_training_amd import (
    FlatParamHandle,
    FSDPConfig,
    GradScaler,
    GradScalerConfig,
    GroupHandle,
    MixedPrecisionConfig,
    OptimizerConfig,
    ShardedOptimizer,
    collect_flat_shard_payload,
    load_flat_shard_checkpoint,
    write_checkpoint,
)
from hybrid_training_amd.host_staging import HostStream
from hybrid_training_amd.optim import NORM_PARTIALS_ATTR, gradient_norm_pass

pytestmark = pytest.mark.gpu

SHAPES = [("a", (300, 77)), ("b", (301,)), ("c", (64, 33)), ("d", (9,))]
TOTAL = 300 * 77 + 301 + 64 * 33 + 9


def _bits(t: torch.Tensor) -> np.ndarray:
    host = t.detach().reshape(-1).cpu()
    width = {8: torch.int64, 4: torch.int32, 2: torch.int16}[host.element_size()]
    return host.view(width).numpy()


def _named(device, seed=5):
    gen = torch.Generator(device=device).manual_seed(seed)
    return [(n, nn.Parameter(torch.randn(s, device=device, generator=gen))) for n, s in SHAPES]


def _handles(named, group, device, offload, mp=None):
    return [FlatParamHandle(named, None, GroupHandle.local_view("shard", group, r),
                            FSDPConfig(cpu_offload_params=offload), mp or MixedPrecisionConfig(), device,
                            keep_originals=True) for r in range(group)]


@pytest.fixture
def small_chunks(monkeypatch):
    monkeypatch.setattr(HostStream, "chunk_elems", 4096)


@pytest.mark.parametrize("mixed", [False, True], ids=["fp32", "bf16_compute"])
@pytest.mark.parametrize("group", [1, 3])
def test_offloaded_handle_is_bitwise_the_hbm_handle(device, small_chunks, group, mixed):
    mp = (MixedPrecisionConfig(enabled=True, param_dtype="bfloat16", reduce_dtype="float32", master_dtype="float32")
          if mixed else MixedPrecisionConfig())
    named = _named(device)
    hbm = _handles(named, group, device, False, mp)
    off = _handles(named, group, device, True, mp)
    for a, b in zip(hbm, off):
        assert b.flat_param.device.type == "cpu" and b.flat_param.is_pinned()
        assert b.device == a.device == device
        assert np.array_equal(_bits(a.flat_param), _bits(b.flat_param))
        assert b.flat_param.gradient_norm_scale_runs == a.flat_param.gradient_norm_scale_runs
        assert b.memory_summary() == a.memory_summary()
    # gather (the all-gather's local side) and unpack from host shards
    full_a = hbm[0].gather_full([h.flat_param for h in hbm] if group > 1 else None)
    full_b = off[0].gather_full([h.flat_param for h in off] if group > 1 else None)
    assert full_b.device == device and np.array_equal(_bits(full_a), _bits(full_b))
    ta = hbm[0].full_tensors([h.flat_param for h in hbm] if group > 1 else None)
    tb = off[0].full_tensors([h.flat_param for h in off] if group > 1 else None)
    for name, _ in SHAPES:
        assert tb[name].device == device and np.array_equal(_bits(ta[name]), _bits(tb[name]))
    # the gradient shard comes back in pinned host memory with its norm partials
    gen = torch.Generator(device=device).manual_seed(3)
    grads = [torch.randn(hbm[0].padded_numel, device=device, generator=gen).to(full_a.dtype) for _ in range(group)]
    for r, (a, b) in enumerate(zip(hbm, off)):
        ga = a.reduce_scatter_gradient(grads[r], peer_grads=grads if group > 1 else None)
        gb = b.reduce_scatter_gradient(grads[r], peer_grads=grads if group > 1 else None)
        assert gb.device.type == "cpu" and gb.is_pinned()
        assert np.array_equal(_bits(ga), _bits(gb)), r
        record = getattr(gb, NORM_PARTIALS_ATTR)
        assert record.data_ptr == gb.data_ptr() and record.version == gb._version
        for key, partials in getattr(ga, NORM_PARTIALS_ATTR).segments.items():
            assert partials.device == device and torch.equal(partials, record.segments[key]), (r, key)
    # pieces: copied out on the device, and written back into a host shard
    for a, b in zip(hbm, off):
        pa, pb = a.local_pieces(), b.local_pieces()
        assert [(p.name, p.offset, p.length) for p in pa] == [(p.name, p.offset, p.length) for p in pb]
        for x, y in zip(pa, pb):
            assert np.array_equal(_bits(x.data), _bits(y.data))
    other = _named(device, seed=99)
    for a, b in zip(hbm, off):
        a.load_local_pieces(dict((n, p.detach()) for n, p in other))
        b.load_local_pieces(dict((n, p.detach()) for n, p in other))
        assert b.flat_param.device.type == "cpu"
        assert np.array_equal(_bits(a.flat_param), _bits(b.flat_param))
    # the padding of a host gradient shard is zeroed like a device one
    last_a, last_b = hbm[-1], off[-1]
    if last_a.padding:
        ga = torch.ones(last_a.shard_numel, device=device)
        gb = torch.ones(last_b.shard_numel).pin_memory()
        last_a.zero_padding_region(ga)
        last_b.zero_padding_region(gb)
        assert np.array_equal(_bits(ga), _bits(gb)) and float(gb[-last_b.padding:].abs().sum()) == 0.0


@pytest.mark.parametrize("name", ["adamw", "sgd"])
@pytest.mark.parametrize("defer_clip", [False, True])
def test_offloaded_fsdp_step_matches_reference_offload_and_oracle(device, small_chunks, name, defer_clip):
    """The reference's offload test (one step of an FSDP unit with and without
    ``cpu_offload_params`` gives the same gradient and the same weights), over three
    clipped steps, with the oracle for every element."""
    named = _named(device)
    lr = 3e-4 if name == "adamw" else 0.05
    config = (OptimizerConfig(learning_rate=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1) if name == "adamw"
              else OptimizerConfig(name="sgd", learning_rate=lr, momentum=0.9, weight_decay=0.01))
    runs = []
    for offload in (False, True):
        handle = _handles(named, 1, device, offload)[0]
        opt = ShardedOptimizer([handle.flat_param], config, norm_group=GroupHandle.trivial(), device=device,
                               defer_clip=defer_clip)
        runs.append((handle, opt))
    shard = runs[0][0].shard_numel
    P = runs[0][0].flat_param.detach().cpu().numpy().copy()
    M, V = np.zeros(shard, np.float32), np.zeros(shard, np.float32)
    gen = torch.Generator(device=device).manual_seed(8)
    for step in range(1, 4):
        grad_full = torch.randn(shard, device=device, generator=gen) * 0.1  # norm ~ 16: clipped
        norms = []
        for handle, opt in runs:
            handle.flat_param.grad = handle.reduce_scatter_gradient(grad_full)
            norms.append(float(opt.clip_grad_norm(1.0)))
            opt.step()
        assert norms[0] == norms[1], step
        (ha, oa), (hb, ob) = runs
        assert hb.flat_param.device.type == "cpu"
        assert np.array_equal(_bits(ha.flat_param), _bits(hb.flat_param)), step
        assert np.array_equal(_bits(ha.flat_param.grad), _bits(hb.flat_param.grad)), step
        mul = oracle.clip_multiplier(norms[0], 1.0)
        assert mul < 1.0
        g = grad_full.cpu().numpy()
        if name == "adamw":
            sc = oracle.adamw_scalars(lr=lr, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=float(step))
            oracle.adamw_step(P, g, M, V, sc, grad_mul=mul)
        else:
            oracle.sgd_step(P, g, M, lr=lr, momentum=0.9, weight_decay=0.01, first=step == 1, grad_mul=mul)
        assert np.array_equal(_bits(hb.flat_param), P.view(np.int32)), step
        for (handle, opt) in runs:
            opt.zero_grad()
    sa, sb = runs[0][1].state_dict()["state"], runs[1][1].state_dict()["state"]
    for key, value in sa[0].items():
        if torch.is_tensor(value):
            assert np.array_equal(_bits(value), _bits(sb[0][key])), key
    state = runs[1][1].inner.state[runs[1][0].flat_param]
    buffers = [state["exp_avg"], state["exp_avg_sq"]] if name == "adamw" else [state["momentum_buffer"]]
    for b in buffers:
        assert b.device.type == "cpu" and b.is_pinned()
    assert np.array_equal(_bits(buffers[0]), M.view(np.int32))
    if name == "adamw":
        assert np.array_equal(_bits(buffers[1]), V.view(np.int32))


@pytest.mark.parametrize("case", range(12))
def test_random_host_resident_parameters(device, monkeypatch, case):
    """Host-resident parameters (all or some of an optimizer's) with random sizes, chunk
    sizes, fp32 / bf16 / fp16 masters, AdamW or SGD, eager or deferred clip, state
    offload on or off, and pinned or pageable host memory (the reference keeps an
    offloaded shard in pageable memory): three steps bitwise those of the same parameters
    in HBM, the returned norms, ``.grad`` and the state included."""
    rng = np.random.default_rng(7000 + case)
    monkeypatch.setattr(HostStream, "chunk_elems", int(rng.choice([1000, 4096, 65536, 1 << 25])))
    sizes = [int(rng.integers(1, 150_000)) for _ in range(int(rng.integers(1, 5)))]
    hosted = [bool(rng.integers(0, 2)) for _ in sizes]
    hosted[0] = True
    adamw = bool(rng.integers(0, 2))
    defer = bool(rng.integers(0, 2))
    state_offload = bool(rng.integers(0, 2))
    pinned = bool(rng.integers(0, 2))
    host_of = (lambda t: t.cpu().pin_memory()) if pinned else (lambda t: t.cpu())
    dtype = [torch.float32, torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 4))]
    config = ({"name": "adamw", "learning_rate": 3e-4, "betas": (0.9, 0.95), "weight_decay": 0.1, "eps": 1e-4}
              if adamw else {"name": "sgd", "learning_rate": 0.05, "momentum": 0.9, "weight_decay": 0.01})
    gen = torch.Generator(device=device).manual_seed(case)
    init = [torch.randn(n, device=device, generator=gen).to(dtype) for n in sizes]
    context = (f"case {case}: sizes {sizes}, hosted {hosted}, {dtype}, adamw {adamw}, defer {defer}, "
               f"state offload {state_offload}, pinned {pinned}, chunk {HostStream.chunk_elems}")
    runs = []
    for host in (False, True):
        params = [nn.Parameter(host_of(t) if host and h else t.clone()) for t, h in zip(init, hosted)]
        opt = ShardedOptimizer(params, OptimizerConfig(**{**config, "cpu_offload_state": state_offload}),
                               norm_group=GroupHandle.trivial(), device=device, defer_clip=defer)
        runs.append((params, opt))
    for step in range(3):
        grads = [(torch.randn(n, device=device, generator=gen) * 0.1).to(dtype) for n in sizes]
        norms = []
        for params, opt in runs:
            for p, g in zip(params, grads):
                p.grad = host_of(g) if p.device.type == "cpu" else g.clone()
            norms.append(float(opt.clip_grad_norm(0.5)))
            opt.step()
        assert norms[0] == norms[1], (context, step)
        for k, (a, b) in enumerate(zip(runs[0][0], runs[1][0])):
            assert b.device.type == ("cpu" if hosted[k] else "cuda")
            assert np.array_equal(_bits(a), _bits(b)), (context, step, k)
            assert np.array_equal(_bits(a.grad), _bits(b.grad)), (context, step, k)
    saved = [opt.state_dict()["state"] for _, opt in runs]
    for index, entry in saved[0].items():
        for key, value in entry.items():
            if torch.is_tensor(value):
                assert np.array_equal(_bits(value), _bits(saved[1][index][key])), (context, index, key)
    for k, p in enumerate(runs[1][0]):
        key = runs[1][1].inner.param_groups[0]["params"][k]
        for value in runs[1][1].inner.state[key].values():
            if torch.is_tensor(value) and value.dim() > 0:
                assert value.device.type == ("cpu" if hosted[k] or state_offload else "cuda"), (context, k)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_host_gradient_norm_at_every_alignment(device, monkeypatch, dtype):
    """Segments of host gradients starting at every element offset from a 16-byte
    boundary, several staged chunks long, with weights and a pending unscale: the same
    fp64 sum, norm and clip multiplier, bit for bit, as the same bytes in HBM at the
    same alignment, and the partials a tagged pass leaves are the device pass's."""
    monkeypatch.setattr(HostStream, "chunk_elems", 3 * 65536 + 5)  # rounds to 3 norm chunks
    per16 = 16 // torch.empty(0, dtype=dtype).element_size()
    gen = torch.Generator(device=device).manual_seed(2)
    for shift in range(per16):
        n = 5 * 65536 + 77
        base = torch.randn(n + per16, device=device, generator=gen).to(dtype)
        dev = base[shift : shift + n]
        host = base.cpu().pin_memory()[shift : shift + n]
        assert (dev.data_ptr() - host.data_ptr()) % 16 == 0
        segments_dev = [(dev, 0, n, 1.0), (dev, 1000, 70_000, 0.5), (dev, 3, 140_001, 2.0)]
        segments_host = [(host, o, k, w) for _, o, k, w in segments_dev]
        for unscale in (None, 0.37):
            if unscale is not None:
                setattr(dev, "_hbt_pending_unscale", unscale)
                setattr(host, "_hbt_pending_unscale", unscale)
            a = gradient_norm_pass(segments_dev, device, max_norm=1.0, tag=True)
            b = gradient_norm_pass(segments_host, device, max_norm=1.0, tag=True)
            assert float(a.sum) == float(b.sum) and float(a.norm) == float(b.norm), (shift, unscale)
            assert float(a.grad_mul) == float(b.grad_mul) and int(a.nonfinite) == int(b.nonfinite) == 0
        ra, rb = getattr(dev, NORM_PARTIALS_ATTR), getattr(host, NORM_PARTIALS_ATTR)
        assert rb.data_ptr == host.data_ptr()
        assert ra.segments.keys() == rb.segments.keys() == {(0, n)}
        assert torch.equal(ra.segments[(0, n)], rb.segments[(0, n)]), shift


@pytest.mark.parametrize("defer_unscale", [False, True])
def test_scaler_on_host_gradients(device, small_chunks, defer_unscale):
    """Eager ``unscale_`` (the reference's in-place ``grad.mul_``) and the overflow check
    on pinned host gradients give the device path's bits; an inf skips the step on both."""
    gen = torch.Generator(device=device).manual_seed(4)
    sizes = [9_000, 33, 20_000]
    init = [torch.randn(n, device=device, generator=gen) for n in sizes]
    runs = []
    for host in (False, True):
        params = [nn.Parameter(t.cpu().pin_memory() if host else t.clone()) for t in init]
        opt = ShardedOptimizer(params, OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                               norm_group=GroupHandle.trivial(), device=device)
        scaler = GradScaler(GradScalerConfig(enabled=True, init_scale=1000.0), GroupHandle.trivial(), device,
                            defer_unscale=defer_unscale)
        runs.append((params, opt, scaler))
    for step in range(3):
        grads = [torch.randn(n, device=device, generator=gen) * 300.0 for n in sizes]
        if step == 1:
            grads[2][123] = float("inf")
        for params, opt, scaler in runs:
            for p, g in zip(params, grads):
                p.grad = g.cpu().pin_memory() if p.device.type == "cpu" else g.clone()
            found = scaler.unscale_(params)
            opt.clip_grad_norm(1.0)
            assert bool(found) == (step == 1)
            assert scaler.step(opt, params) == (step != 1)
            scaler.update()
        for a, b in zip(runs[0][0], runs[1][0]):
            assert np.array_equal(_bits(a), _bits(b)), step
            assert np.array_equal(_bits(a.grad), _bits(b.grad)), step
        assert runs[0][2].scale_value == runs[1][2].scale_value


def test_offloaded_checkpoint_round_trip(device, tmp_path, small_chunks):
    """A checkpoint written from host-resident shards (and their host state) loads back
    bitwise into offloaded and into in-HBM readers at another width."""
    named = _named(device)
    writers = _handles(named, 2, device, True)
    opts = [ShardedOptimizer([h.flat_param], OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                             norm_group=GroupHandle.local_view("world", 2, r), device=device)
            for r, h in enumerate(writers)]
    gen = torch.Generator(device=device).manual_seed(1)
    for _ in range(2):
        for h, opt in zip(writers, opts):
            h.flat_param.grad = (torch.randn(h.shard_numel, device=device, generator=gen) * 1e-2).cpu().pin_memory()
            opt.step()
    shards = [(r, *collect_flat_shard_payload(h, rank=r, optimizer=opt)) for r, (h, opt) in
              enumerate(zip(writers, opts))]
    path = write_checkpoint(tmp_path, 2, shards, topology={"fsdp": 2})
    flat = torch.cat([h.flat_param.detach() for h in writers])[:TOTAL]
    m = torch.cat([o.inner.state[h.flat_param]["exp_avg"] for h, o in zip(writers, opts)])[:TOTAL]
    for offload in (True, False):
        readers = _handles(_named(device, seed=77), 3, device, offload)
        for r, h in enumerate(readers):
            opt = ShardedOptimizer([h.flat_param], OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                                   norm_group=GroupHandle.local_view("world", 3, r), device=device)
            load_flat_shard_checkpoint(path, h, optimizer=opt)
            assert (h.flat_param.device.type == "cpu") == offload
            start = r * h.shard_numel
            valid = max(0, min(h.shard_numel, TOTAL - start))
            assert np.array_equal(_bits(h.flat_param[:valid]), _bits(flat[start : start + valid])), (offload, r)
            state = opt.inner.state[h.flat_param]
            assert (state["exp_avg"].device.type == "cpu") == offload
            assert np.array_equal(_bits(state["exp_avg"][:valid]), _bits(m[start : start + valid])), (offload, r)


@pytest.mark.parametrize("mixed", [False, True], ids=["fp32", "fp16_compute"])
def test_offloaded_no_sync_and_storage_cycle(device, small_chunks, mixed):
    """``no_sync`` accumulation (``fsdp.py:738-749``) and the gathered buffer's storage
    cycle (``unshard`` / ``reshard`` / ``refill``, ``fsdp.py:624-701``) on an offloaded
    unit at G = 3: every gradient shard and every refilled buffer is the in-HBM unit's,
    bitwise; with fp16 compute the loss-scaled engine tail (eager unscale, clip, AdamW)
    follows as well."""
    mp = (MixedPrecisionConfig(enabled=True, param_dtype="float16", reduce_dtype="float32", master_dtype="float32",
                               scaler=GradScalerConfig(enabled=True, init_scale=1024.0))
          if mixed else MixedPrecisionConfig())
    named = _named(device, seed=6)
    group = 3
    runs = []
    for offload in (False, True):
        handles = _handles(named, group, device, offload, mp)
        opts = [ShardedOptimizer([h.flat_param], OptimizerConfig(learning_rate=1e-3, weight_decay=0.01),
                                 norm_group=GroupHandle.local_view("world", group, r), device=device)
                for r, h in enumerate(handles)]
        scaler = GradScaler(GradScalerConfig(enabled=mixed, init_scale=1024.0), GroupHandle.trivial(), device)
        runs.append((handles, opts, scaler))
    gen = torch.Generator(device=device).manual_seed(13)
    padded = runs[0][0][0].padded_numel
    for step in range(2):
        compute = torch.float16 if mixed else torch.float32
        micro = [[(torch.randn(padded, device=device, generator=gen) * 0.05).to(compute) for _ in range(group)]
                 for _ in range(3)]
        shards = []
        for handles, opts, scaler in runs:
            fulls = []
            for r, h in enumerate(handles):
                full = h.unshard([x.flat_param for x in handles])
                h.reshard()
                assert full.untyped_storage().nbytes() == 0
                h.refill(full, [x.flat_param for x in handles])
                fulls.append(full)
                h.set_accumulate_without_reduction(True)
                for grads in micro[:-1]:
                    assert h.reduce_scatter_gradient(grads[r], peer_grads=grads) is None
                h.set_accumulate_without_reduction(False)
                h.flat_param.grad = h.reduce_scatter_gradient(micro[-1][r], peer_grads=micro[-1])
            for h, opt in zip(handles, opts):
                params = [h.flat_param]
                scaler.unscale_(params)
                opt.clip_grad_norm(0.5)
                scaler.step(opt, params, already_unscaled=True)
                opt.zero_grad(set_to_none=False)
            scaler.update()
            shards.append(([_bits(h.flat_param) for h in handles], [_bits(f) for f in fulls]))
        for r in range(group):
            assert np.array_equal(shards[0][0][r], shards[1][0][r]), (step, r)
            assert np.array_equal(shards[0][1][r], shards[1][1][r]), (step, r)
        for h in runs[1][0]:
            assert h.flat_param.device.type == "cpu" and not h.has_pending_accumulation


def test_parameter_and_gradient_must_live_together(device):
    """A host-resident parameter steps with a host gradient; torch itself refuses a device
    gradient on it, a missing gradient leaves it untouched, and a gradient that is not
    dense is refused before any copy or launch, with the reference's error class."""
    from hybrid_training_amd.errors import ShardingError

    host = nn.Parameter(torch.zeros(1000).pin_memory())
    opt = ShardedOptimizer([host], OptimizerConfig(learning_rate=1e-3), norm_group=GroupHandle.trivial(),
                           device=device)
    host.grad = torch.ones(1000).pin_memory()
    opt.step()  # fine
    assert host.device.type == "cpu" and float(host.detach().abs().sum()) > 0
    with pytest.raises(RuntimeError):
        host.grad = torch.ones(1000, device=device)  # torch itself refuses the assignment
    dev = nn.Parameter(torch.zeros(1000, device=device))
    opt2 = ShardedOptimizer([dev], OptimizerConfig(learning_rate=1e-3), norm_group=GroupHandle.trivial(), device=device)
    dev.grad = torch.ones(1000, device=device)
    opt2.step()
    before = host.detach().clone()
    bad = ShardedOptimizer([host], OptimizerConfig(learning_rate=1e-3), norm_group=GroupHandle.trivial(), device=device)
    host.grad = None
    bad.step()  # no gradient: nothing to do
    assert torch.equal(host.detach(), before)
    with pytest.raises(ShardingError, match="dense"):
        host.grad = torch.ones(2000).pin_memory()[::2]
        bad.step()
