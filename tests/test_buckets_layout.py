"""DDP bucket layout rule (host logic, no GPU).

The rule is ``parallel/ddp.py:397-463``: reverse registration order, close a bucket
when the next parameter would exceed ``int(cap_mb * 2**20)`` bytes or when dtype or
device changes.  Pinned by the reference's invariants
(``tests/unit/test_single_process_components.py:145-178``) and, for GPT-2 small at
the 25 MiB default, by the bucket table derived from the same rule: 17 buckets,
bucket 0 = the 11 tensors ``ln_f.bias`` .. ``h.11.attn.c_attn.bias`` (5,318,400
elements), bucket 16 = ``wte`` alone (38,597,376 elements).
"""

from __future__ import annotations

import torch

import oracle
from hybrid_training_amd import build_buckets

from .model_shapes import GPT2_SMALL


def _meta_params(named_shapes, dtype=torch.float32):
    return [(n, torch.nn.Parameter(torch.empty(s, dtype=dtype, device="meta"))) for n, s in named_shapes]


def test_gpt2_small_buckets_at_25_mib():
    named = _meta_params(GPT2_SMALL)
    buckets = build_buckets(named, 25.0)
    assert sum(p.numel() for _, p in named) == 124_439_808
    assert len(buckets) == 17
    first = buckets[0].layout
    assert len(first.parameter_names) == 11 and first.total_numel == 5_318_400
    assert first.parameter_names[0] == "ln_f.bias" and first.parameter_names[-1] == "h.11.attn.c_attn.bias"
    last = buckets[-1].layout
    assert last.parameter_names == ("wte.weight",) and last.total_numel == 38_597_376
    middle = [b.layout.total_numel for b in buckets[1:-1]]
    assert min(middle) == 4_725_504 and max(middle) == 6_495_744
    expected = oracle.bucket_layout([(n, p.numel(), 4) for n, p in named], int(25.0 * 2**20))
    assert [[(n, o, k) for n, o, k in b] for b in expected] == [
        list(zip(b.layout.parameter_names, b.layout.offsets, b.layout.numels)) for b in buckets
    ]


def test_reverse_order_contiguity_and_exactly_once():
    named = _meta_params([("a", (8, 16)), ("b", (16,)), ("c", (16, 16)), ("d", (16,)), ("e", (4, 16)), ("f", (4,))])
    for cap in (1e-6, 0.001, 0.002, 100.0):
        buckets = build_buckets(named, cap)
        flat = [n for b in buckets for n in b.layout.parameter_names]
        assert flat == [n for n, _ in reversed(named)]
        for b in buckets:
            cursor = 0
            for off, numel in zip(b.layout.offsets, b.layout.numels):
                assert off == cursor
                cursor += numel
            assert cursor == b.layout.total_numel
    assert len(build_buckets(named, 100.0)) == 1
    assert len(build_buckets(named, 1e-6)) == len(named)


def test_dtype_change_closes_a_bucket():
    named = _meta_params([("a", (4,)), ("b", (4,))]) + _meta_params([("c", (4,))], torch.bfloat16)
    buckets = build_buckets(named, 100.0)
    assert [b.layout.parameter_names for b in buckets] == [("c",), ("b", "a")]
    assert buckets[0].layout.dtype_str == "torch.bfloat16"
    assert buckets[1].num_bytes() == 32
