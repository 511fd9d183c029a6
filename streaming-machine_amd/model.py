"""Synthetic float weights of GPT-2 124M shape (no network here, so no pretrained checkpoint).

The draw is fixed so every machine produces the same bits: one numpy PCG64 generator, default_rng(seed),
walks the state dict in Hugging Face GPT2LMHeadModel order and draws float64 normals that are cast to float32
(the checkpoint dtype).  Weights, biases and layer-norm offsets are N(0, 0.02); layer-norm gains are
1 + N(0, 0.02) so that layer norm keeps unit scale (a literal N(0, 0.02) gain would shrink every normalised
row about fifty times and flatten the machine's numbers).
"""
from __future__ import annotations

import numpy as np

GPT2_SHAPE = dict(n_layer=12, d=768, n_head=12, d_ff=3072, vocab=50257, n_ctx=1024)


def random_gpt2(seed: int = 0, vocab: int = 50257, n_ctx: int = 1024, n_layer: int = 12, std: float = 0.02) -> dict:
    """HF-named float32 state dict of a GPT-2 (d=768, 12 heads, FFN 3072) with the given vocabulary size."""
    rng = np.random.default_rng(seed)
    d, f = 768, 3072

    def nrm(*shape):
        return (rng.standard_normal(shape) * std).astype(np.float32)

    def gain(n):
        return (1.0 + rng.standard_normal(n) * std).astype(np.float32)

    sd = {"transformer.wte.weight": nrm(vocab, d), "transformer.wpe.weight": nrm(n_ctx, d)}
    for l in range(n_layer):
        p = f"transformer.h.{l}."
        sd[p + "ln_1.weight"] = gain(d)
        sd[p + "ln_1.bias"] = nrm(d)
        sd[p + "attn.c_attn.weight"] = nrm(d, 3 * d)
        sd[p + "attn.c_attn.bias"] = nrm(3 * d)
        sd[p + "attn.c_proj.weight"] = nrm(d, d)
        sd[p + "attn.c_proj.bias"] = nrm(d)
        sd[p + "ln_2.weight"] = gain(d)
        sd[p + "ln_2.bias"] = nrm(d)
        sd[p + "mlp.c_fc.weight"] = nrm(d, f)
        sd[p + "mlp.c_fc.bias"] = nrm(f)
        sd[p + "mlp.c_proj.weight"] = nrm(f, d)
        sd[p + "mlp.c_proj.bias"] = nrm(d)
    sd["transformer.ln_f.weight"] = gain(d)
    sd["transformer.ln_f.bias"] = nrm(d)
    return sd


def prompt_ids(seed: int, n: int, vocab: int = 50257) -> list:
    """Uniform random token ids from default_rng(seed)."""
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]
