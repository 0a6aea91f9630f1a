"""Parameter shapes of the models the benchmark configurations name (synthetic weights only).

* The reference's test MLP ``14-25x3-7`` (``tests/distributed/test_fsdp.py:42-46``) and the
  ``Linear(23,32)-ReLU-Linear(32,32)-ReLU-Linear(32,1)`` MLP: both have 1857 parameters.
* GPT-2 small (12 layers, d=768, vocab 50257, 1024 positions): 148 tensors, 124,439,808.
* Llama-3-8B (32 layers, d=4096, ffn 14336, 32 query / 8 key-value heads of 128, vocab
  128256, untied output head): 291 tensors, 8,030,261,248.
* Llama-3-70B (80 layers, d=8192, ffn 28672, 64/8 heads, vocab 128256): 70,553,706,496.
"""

from __future__ import annotations

MLP_1857_REFERENCE = [(25, 14), (25,), (25, 25), (25,), (25, 25), (25,), (7, 25), (7,)]
MLP_23_32_32_1 = [(32, 23), (32,), (32, 32), (32,), (1, 32), (1,)]


def gpt2_small() -> list[tuple[str, tuple[int, ...]]]:
    d, vocab, ctx = 768, 50257, 1024
    named = [("wte.weight", (vocab, d)), ("wpe.weight", (ctx, d))]
    for i in range(12):
        p = f"h.{i}."
        named += [
            (p + "ln_1.weight", (d,)), (p + "ln_1.bias", (d,)),
            (p + "attn.c_attn.weight", (d, 3 * d)), (p + "attn.c_attn.bias", (3 * d,)),
            (p + "attn.c_proj.weight", (d, d)), (p + "attn.c_proj.bias", (d,)),
            (p + "ln_2.weight", (d,)), (p + "ln_2.bias", (d,)),
            (p + "mlp.c_fc.weight", (d, 4 * d)), (p + "mlp.c_fc.bias", (4 * d,)),
            (p + "mlp.c_proj.weight", (4 * d, d)), (p + "mlp.c_proj.bias", (d,)),
        ]
    named += [("ln_f.weight", (d,)), ("ln_f.bias", (d,))]
    return named


GPT2_SMALL = gpt2_small()


def llama3(layers: int, d: int, ffn: int, kv_dim: int, vocab: int) -> list[tuple[str, tuple[int, ...]]]:
    named = [("model.embed_tokens.weight", (vocab, d))]
    for i in range(layers):
        p = f"model.layers.{i}."
        named += [
            (p + "self_attn.q_proj.weight", (d, d)),
            (p + "self_attn.k_proj.weight", (kv_dim, d)),
            (p + "self_attn.v_proj.weight", (kv_dim, d)),
            (p + "self_attn.o_proj.weight", (d, d)),
            (p + "mlp.gate_proj.weight", (ffn, d)),
            (p + "mlp.up_proj.weight", (ffn, d)),
            (p + "mlp.down_proj.weight", (d, ffn)),
            (p + "input_layernorm.weight", (d,)),
            (p + "post_attention_layernorm.weight", (d,)),
        ]
    named += [("model.norm.weight", (d,)), ("lm_head.weight", (vocab, d))]
    return named


LLAMA3_8B = llama3(32, 4096, 14336, 1024, 128256)


def _numel(shape: tuple[int, ...]) -> int:
    n = 1
    for s in shape:
        n *= s
    return n


LLAMA3_70B_TOTAL = sum(_numel(s) for _, s in llama3(80, 8192, 28672, 1024, 128256))
