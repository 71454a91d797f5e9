"""Write the golden fixtures under tests/golden/ (run from the repo root).

The reference (falcons-eyes/cutileGPT) ships no golden vectors and cannot run
here (cuda.tile + CuPy + an NVIDIA GPU), so the fixtures are produced by an
independent implementation of the same architecture: transformers'
``GPT2LMHeadModel`` (gelu_new, layer_norm_epsilon 1e-5, tied embeddings) in
float64 on the CPU, fed the seeded weights below.  Weights: the nano
configuration of the benchmark (3 layers, 3 heads, n_embd 48, vocab 50257,
block 1024), every Linear/embedding weight ~ N(0, 0.02) drawn in a fixed key
order from ``torch.Generator().manual_seed(0)``, biases 0, LayerNorm gamma 1 /
beta 0; token ids ``randint(0, 50257, (1, 64))`` from seed 1.

Fixture ``nano_seed0.npz``: ids, last-position logits (50257 fp64), per-position
argmax, per-position logit sum and absmax, and greedy continuation of 8 tokens.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def nano_weights(seed=0):
    """Seeded nano weights, drawn in the key order of the benchmark recipe."""
    g = torch.Generator().manual_seed(seed)
    L, D, V, BS = 3, 48, 50257, 1024
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float32) * 0.02
    w = {"wte": r(V, D), "wpe": r(BS, D)}
    for i in range(L):
        p = f"h.{i}."
        w[p + "ln_1.weight"] = torch.ones(D); w[p + "ln_1.bias"] = torch.zeros(D)
        w[p + "attn.c_attn.weight"] = r(3 * D, D); w[p + "attn.c_attn.bias"] = torch.zeros(3 * D)
        w[p + "attn.c_proj.weight"] = r(D, D); w[p + "attn.c_proj.bias"] = torch.zeros(D)
        w[p + "ln_2.weight"] = torch.ones(D); w[p + "ln_2.bias"] = torch.zeros(D)
        w[p + "mlp.c_fc.weight"] = r(4 * D, D); w[p + "mlp.c_fc.bias"] = torch.zeros(4 * D)
        w[p + "mlp.c_proj.weight"] = r(D, 4 * D); w[p + "mlp.c_proj.bias"] = torch.zeros(D)
    w["ln_f.weight"] = torch.ones(D); w["ln_f.bias"] = torch.zeros(D)
    return w


def hf_model(w, n_layer, n_head, n_embd, vocab=50257, block=1024):
    from transformers import GPT2Config, GPT2LMHeadModel
    cfg = GPT2Config(vocab_size=vocab, n_positions=block, n_embd=n_embd, n_layer=n_layer,
                     n_head=n_head, activation_function="gelu_new", layer_norm_epsilon=1e-5,
                     resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0, tie_word_embeddings=True)
    m = GPT2LMHeadModel(cfg).eval()
    sd = {"transformer.wte.weight": w["wte"], "transformer.wpe.weight": w["wpe"],
          "transformer.ln_f.weight": w["ln_f.weight"], "transformer.ln_f.bias": w["ln_f.bias"]}
    for i in range(n_layer):
        for name in ("ln_1.weight", "ln_1.bias", "attn.c_attn.bias", "attn.c_proj.bias",
                     "ln_2.weight", "ln_2.bias", "mlp.c_fc.bias", "mlp.c_proj.bias"):
            sd[f"transformer.h.{i}.{name}"] = w[f"h.{i}.{name}"]
        for name in ("attn.c_attn.weight", "attn.c_proj.weight", "mlp.c_fc.weight",
                     "mlp.c_proj.weight"):  # HF Conv1D stores (in, out)
            sd[f"transformer.h.{i}.{name}"] = w[f"h.{i}.{name}"].t().contiguous()
    sd["lm_head.weight"] = w["wte"]
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("attn.bias" in k or "masked_bias" in k for k in missing), (missing, unexpected)
    return m


def main():
    torch.manual_seed(0)
    w = nano_weights(0)
    ids = torch.randint(0, 50257, (1, 64), generator=torch.Generator().manual_seed(1))
    m = hf_model(w, 3, 3, 48).double()
    with torch.no_grad():
        logits = m(ids).logits[0]  # (64, V) fp64
        gen = m.generate(ids[:, :16], max_new_tokens=8, do_sample=False, pad_token_id=0)
    np.savez_compressed(
        os.path.join(HERE, "nano_seed0.npz"),
        ids=ids.numpy(), last_logits=logits[-1].numpy(), argmax=logits.argmax(-1).numpy(),
        row_sum=logits.sum(-1).numpy(), row_absmax=logits.abs().amax(-1).numpy(),
        greedy_prompt=ids[:, :16].numpy(), greedy_out=gen.numpy())
    print("wrote", os.path.join(HERE, "nano_seed0.npz"))


if __name__ == "__main__":
    sys.exit(main())
