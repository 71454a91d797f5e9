"""CPU restatement of the reference GPT-2 forward — TEST INFRASTRUCTURE ONLY.

Each function cites the reference file:line (relative to the falcons-eyes/cutileGPT
checkout) whose arithmetic it restates.  Arithmetic runs in ``flow.compute``
(float64 or float32) on CPU tensors; ``Flow`` describes where activations are
stored and in which dtype, so that the same restatement can model

* ``fp64``      the exact result (used to judge error budgets),
* ``fp32``      the reference's fp32 path with true fp32 products,
* ``bf16_ref``  the reference's own dtype flow when its tensors are bf16: every
                kernel computes in fp32 and stores its output in the input dtype
                (``kernels/linear.py:109``, ``kernels/layernorm.py:74``,
                ``kernels/attention.py:109,115``), residual adds in bf16
                (``models/gpt.py:155,174``), logits in bf16 (``linear.py:146``),
* ``bf16``      the HIP path's flow: bf16 operands for every matrix product,
                c_proj outputs stored bf16 (as the reference stores them) and
                added to an fp32 residual stream, GELU fused into the
                up-projection (one rounding), fp32 logits.

Only ``tests/``, ``__graft_entry__.smoke`` and ``bench.py``'s CPU-baseline leg use
this module.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional

import torch

# gelu.py:15-17
SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
GELU_COEF = 0.044715
# layernorm.py:81 (default eps of cutile_layer_norm)
LN_EPS = 1e-5


@dataclass(frozen=True)
class Flow:
    name: str
    compute: torch.dtype      # arithmetic dtype inside every op
    act: torch.dtype          # storage of LN outputs, QKV, attention output, GELU output
    resid: torch.dtype        # storage of the residual stream x
    delta: torch.dtype        # storage of c_proj outputs before the residual add
    logits: torch.dtype       # storage of the logits
    p: torch.dtype            # dtype P is rounded to before the P.V product
    fused_gelu: bool          # GELU applied to the unrounded c_fc accumulator


FLOWS: Dict[str, Flow] = {
    "fp64": Flow("fp64", torch.float64, torch.float64, torch.float64, torch.float64,
                 torch.float64, torch.float64, True),
    "fp32": Flow("fp32", torch.float32, torch.float32, torch.float32, torch.float32,
                 torch.float32, torch.float32, False),
    "bf16_ref": Flow("bf16_ref", torch.float32, torch.bfloat16, torch.bfloat16,
                     torch.bfloat16, torch.bfloat16, torch.bfloat16, False),
    "bf16": Flow("bf16", torch.float32, torch.bfloat16, torch.float32, torch.bfloat16,
                 torch.float32, torch.bfloat16, True),
}


def round_to(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Round ``t`` to ``dtype`` storage and bring it back to ``t.dtype`` (RNE)."""
    if dtype == t.dtype or dtype in (torch.float64,) and t.dtype == torch.float32:
        return t
    return t.to(dtype).to(t.dtype)


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """tanh-approximate GELU, ``0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))``.

    Restates ``cutile_gpt/kernels/gelu.py:35-38`` (constants ``:15-17``).
    """
    inner = SQRT_2_OVER_PI * (x + GELU_COEF * (x * x * x))
    return 0.5 * x * (1.0 + torch.tanh(inner))


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
               eps: float = LN_EPS) -> torch.Tensor:
    """LayerNorm over the last axis with biased variance.

    Restates ``cutile_gpt/kernels/layernorm.py:43-74``: mean = sum/N,
    var = sum(x^2)/N - mean^2, rstd = 1/sqrt(var + eps), y = (x-mean)*rstd*w + b.
    """
    n = x.shape[-1]
    mean = x.sum(-1, keepdim=True) / n
    var = (x * x).sum(-1, keepdim=True) / n - mean * mean
    rstd = 1.0 / torch.sqrt(var + eps)
    return (x - mean) * rstd * weight + bias


def linear(x: torch.Tensor, weight: torch.Tensor,
           bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``y = x @ weight.T (+ bias)`` with ``weight`` laid out (out, in).

    Restates ``cutile_gpt/kernels/linear.py:112-222`` (the kernels multiply by the
    cached transpose ``weight.T``, ``:138-143,196-201``, and add the bias after the
    K loop, ``:104-107``).
    """
    y = x @ weight.t()
    if bias is not None:
        y = y + bias
    return y


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     p_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Causal softmax attention on (B, H, T, hd) tensors.

    Restates ``cutile_gpt/kernels/attention.py:24-116``: scores scaled by
    1/sqrt(hd) (``:154``), key j visible to query i iff j <= i (``:90-94``),
    softmax over visible keys, P rounded to the input dtype before the P.V
    product (``:109``) while the normaliser sums unrounded P (``:100-103``).
    The online (running-max) formulation of the kernel is algebraically this
    two-pass softmax.
    """
    hd = q.shape[-1]
    t_q, t_k = q.shape[-2], k.shape[-2]
    scale = 1.0 / math.sqrt(hd)
    s = (q @ k.transpose(-1, -2)) * scale
    # query i sits at absolute position (t_k - t_q + i): the prefill case has
    # t_q == t_k; a decode step (t_q == 1) sees every cached key.
    qi = torch.arange(t_q).unsqueeze(1) + (t_k - t_q)
    kj = torch.arange(t_k).unsqueeze(0)
    s = s.masked_fill(kj > qi, float("-inf"))
    m = s.amax(-1, keepdim=True)
    p = torch.exp(s - m)
    l = p.sum(-1, keepdim=True)
    if p_dtype is not None:
        p = round_to(p, p_dtype)
    return (p @ v) / l


def embedding(idx: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Row gather ``weight[idx]``; restates ``cutile_gpt/kernels/embedding.py:23-51``."""
    return weight[idx]


def _n_layer(w: Dict[str, torch.Tensor]) -> int:
    return len({k.split(".")[1] for k in w if k.startswith("h.")})


def gpt_forward(w: Dict[str, torch.Tensor], idx: torch.Tensor, n_head: int,
                flow: Flow = FLOWS["fp32"]) -> torch.Tensor:
    """Pre-LN GPT-2 forward returning logits (B, T, V) in ``flow.compute``.

    Restates ``cutile_gpt/models/gpt.py:95-183``: x = wte[idx] + wpe[pos];
    per layer x += c_proj(attn(ln_1(x))); x += mlp.c_proj(gelu(c_fc(ln_2(x))));
    logits = ln_f(x) @ lm_head.weight.T with no LM-head bias.  ``w`` uses the
    reference's weight-dict keys (``models/gpt.py:45-81``), Linear weights (out, in).
    """
    c = flow.compute

    def W(key: str) -> torch.Tensor:
        return w[key].to(c)

    B, T = idx.shape
    D = w["wte"].shape[1]
    hd = D // n_head
    # gpt.py:110-113
    tok = embedding(idx, W("wte"))
    pos = embedding(torch.arange(T), W("wpe"))
    x = round_to(tok + pos.unsqueeze(0), flow.resid)
    for i in range(_n_layer(w)):
        p = f"h.{i}."
        # gpt.py:120-137
        h = round_to(layer_norm(x, W(p + "ln_1.weight"), W(p + "ln_1.bias")), flow.act)
        qkv = round_to(linear(h, W(p + "attn.c_attn.weight"), W(p + "attn.c_attn.bias")), flow.act)
        q, k, v = qkv.split(D, dim=2)
        q, k, v = (t.reshape(B, T, n_head, hd).transpose(1, 2) for t in (q, k, v))
        # gpt.py:140-155
        a = round_to(causal_attention(q, k, v, flow.p), flow.act)
        a = a.transpose(1, 2).reshape(B, T, D)
        d = round_to(linear(a, W(p + "attn.c_proj.weight"), W(p + "attn.c_proj.bias")), flow.delta)
        x = round_to(x + d, flow.resid)
        # gpt.py:158-174
        h = round_to(layer_norm(x, W(p + "ln_2.weight"), W(p + "ln_2.bias")), flow.act)
        f = linear(h, W(p + "mlp.c_fc.weight"), W(p + "mlp.c_fc.bias"))
        if not flow.fused_gelu:
            f = round_to(f, flow.act)
        g = round_to(gelu_tanh(f), flow.act)
        d = round_to(linear(g, W(p + "mlp.c_proj.weight"), W(p + "mlp.c_proj.bias")), flow.delta)
        x = round_to(x + d, flow.resid)
    # gpt.py:177-183
    h = round_to(layer_norm(x, W("ln_f.weight"), W("ln_f.bias")), flow.act)
    return round_to(linear(h, W("lm_head.weight")), flow.logits)


@torch.inference_mode()
def generate(w: Dict[str, torch.Tensor], idx: torch.Tensor, n_head: int, max_new_tokens: int,
             flow: Flow = FLOWS["fp32"], block_size: int = 1024) -> torch.Tensor:
    """Greedy autoregressive continuation (the reference's ``top_k=1`` case).

    Restates ``cutile_gpt/models/gpt.py:185-229``: crop the context to the last
    ``block_size`` tokens, run the full forward, take the last position's logits;
    with ``top_k=1`` every token but the argmax is masked to -inf (``:209-213``),
    so the sampled token is the argmax.  Ties resolve to the lowest index.
    """
    for _ in range(max_new_tokens):
        cond = idx if idx.shape[1] <= block_size else idx[:, -block_size:]
        logits = gpt_forward(w, cond, n_head, flow)[:, -1, :]
        nxt = logits.argmax(-1, keepdim=True)
        idx = torch.cat([idx, nxt], dim=1)
    return idx


def init_weights(n_layer: int, n_head: int, n_embd: int, vocab_size: int = 50257,
                 block_size: int = 1024, seed: int = 0, dtype: torch.dtype = torch.float32,
                 scheme: str = "baseline") -> Dict[str, torch.Tensor]:
    """Seeded CPU weights in the reference's weight-dict layout (``models/gpt.py:39-81``).

    ``scheme="baseline"``: every Linear/embedding weight ~ N(0, 0.02), biases 0,
    LayerNorm gamma 1, beta 0 (the benchmark configurations).
    ``scheme="reference"``: as ``models/gpt.py:45-81`` (both c_proj weights scaled
    by 1/sqrt(2 n_layer)).  ``lm_head.weight`` is ``wte`` (tied, ``:81``).
    Draws happen in a fixed key order from ``torch.Generator().manual_seed(seed)``
    in fp32 and are then cast to ``dtype``.
    """
    g = torch.Generator().manual_seed(seed)
    D = n_embd

    def randn(*shape, std=0.02):
        return (torch.randn(*shape, generator=g, dtype=torch.float32) * std).to(dtype)

    proj_std = 0.02 / math.sqrt(2 * n_layer) if scheme == "reference" else 0.02
    w: Dict[str, torch.Tensor] = {}
    w["wte"] = randn(vocab_size, D)
    w["wpe"] = randn(block_size, D)
    for i in range(n_layer):
        p = f"h.{i}."
        w[p + "ln_1.weight"] = torch.ones(D, dtype=dtype)
        w[p + "ln_1.bias"] = torch.zeros(D, dtype=dtype)
        w[p + "attn.c_attn.weight"] = randn(3 * D, D)
        w[p + "attn.c_attn.bias"] = torch.zeros(3 * D, dtype=dtype)
        w[p + "attn.c_proj.weight"] = randn(D, D, std=proj_std)
        w[p + "attn.c_proj.bias"] = torch.zeros(D, dtype=dtype)
        w[p + "ln_2.weight"] = torch.ones(D, dtype=dtype)
        w[p + "ln_2.bias"] = torch.zeros(D, dtype=dtype)
        w[p + "mlp.c_fc.weight"] = randn(4 * D, D)
        w[p + "mlp.c_fc.bias"] = torch.zeros(4 * D, dtype=dtype)
        w[p + "mlp.c_proj.weight"] = randn(D, 4 * D, std=proj_std)
        w[p + "mlp.c_proj.bias"] = torch.zeros(D, dtype=dtype)
    w["ln_f.weight"] = torch.ones(D, dtype=dtype)
    w["ln_f.bias"] = torch.zeros(D, dtype=dtype)
    w["lm_head.weight"] = w["wte"]
    return w
