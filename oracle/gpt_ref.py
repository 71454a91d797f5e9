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
                P rounded per 64-key block relative to the running maximum
                (``kernels/attention.py:96-110``),
* ``bf16``      the HIP path's flow: bf16 operands for every matrix product
                (LN outputs, QKV, attention output, GELU output and P stored
                bf16), c_proj outputs kept fp32 and added to an fp32 residual
                stream, GELU fused into the up-projection (one rounding), fp32
                logits, P rounded per 64-key block relative to a running
                maximum that moves only when a block's maximum exceeds it by
                more than 2^8 (the HIP kernel's lazy rescaling).

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
    # Where P is rounded (only matters when ``p`` is narrower than ``compute``):
    # None = relative to each row's final maximum (two-pass softmax); a number
    # = online softmax over 64-key blocks, relative to the running maximum,
    # which moves to a block's maximum only when that exceeds it by more than
    # this many powers of two (0: every increase, the reference's rule).
    online_lazy: Optional[float] = None


FLOWS: Dict[str, Flow] = {
    "fp64": Flow("fp64", torch.float64, torch.float64, torch.float64, torch.float64,
                 torch.float64, torch.float64, True),
    "fp32": Flow("fp32", torch.float32, torch.float32, torch.float32, torch.float32,
                 torch.float32, torch.float32, False),
    "bf16_ref": Flow("bf16_ref", torch.float32, torch.bfloat16, torch.bfloat16,
                     torch.bfloat16, torch.bfloat16, torch.bfloat16, False, 0.0),
    "bf16": Flow("bf16", torch.float32, torch.bfloat16, torch.float32, torch.float32,
                 torch.float32, torch.bfloat16, True, 8.0),
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


def online_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     p_dtype: Optional[torch.dtype] = None, causal: bool = True,
                     lazy_log2: float = 0.0, block: int = 64) -> torch.Tensor:
    """Causal attention in the online (running-maximum) form of the kernel,
    over key blocks of ``block`` keys taken in order.

    Restates ``cutile_gpt/kernels/attention.py:80-116``: per block, scores are
    scaled into the base-2 domain (scale / ln 2), the running maximum m moves to
    max(m, block maximum), P = 2^(s - m) is summed unrounded into the
    normaliser, rounded to the input dtype (``:109``) and multiplied with V;
    earlier sums are rescaled by 2^(m_old - m_new); the result is divided by
    the normaliser.  ``lazy_log2 > 0`` moves the maximum only when a block's
    maximum exceeds it by more than that many powers of two (P then reaches
    up to 2^lazy_log2; in exact arithmetic nothing changes).
    """
    hd = q.shape[-1]
    t_q, t_k = q.shape[-2], k.shape[-2]
    c = (1.0 / math.sqrt(hd)) / math.log(2.0)
    s_all = q @ k.transpose(-1, -2)
    if causal:
        qi = torch.arange(t_q).unsqueeze(1) + (t_k - t_q)
        kj = torch.arange(t_k).unsqueeze(0)
        s_all = s_all.masked_fill(kj > qi, float("-inf"))
    ninf = float("-inf")
    m = torch.full(q.shape[:-1] + (1,), ninf, dtype=q.dtype)
    l = torch.zeros_like(m)
    acc = torch.zeros(q.shape[:-1] + (v.shape[-1],), dtype=q.dtype)
    for j0 in range(0, t_k, block):
        s = s_all[..., j0:j0 + block]
        mblk = s.amax(-1, keepdim=True) * c
        m_new = torch.where(mblk > m + lazy_log2, mblk, m) if lazy_log2 > 0 else torch.maximum(m, mblk)
        alpha = torch.where(m == ninf, torch.zeros_like(m), torch.exp2(m - m_new))
        p = torch.exp2(s * c - torch.where(m_new == ninf, torch.zeros_like(m_new), m_new))
        l = l * alpha + p.sum(-1, keepdim=True)
        if p_dtype is not None:
            p = round_to(p, p_dtype)
        acc = acc * alpha + p @ v[..., j0:j0 + block, :]
        m = m_new
    return acc / l


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     p_dtype: Optional[torch.dtype] = None, causal: bool = True) -> torch.Tensor:
    """Causal softmax attention on (B, H, T, hd) tensors.

    Restates ``cutile_gpt/kernels/attention.py:24-116``: scores scaled by
    1/sqrt(hd) (``:154``), key j visible to query i iff j <= i (``:90-94``),
    softmax over visible keys, P rounded to the input dtype before the P.V
    product (``:109``) while the normaliser sums unrounded P (``:100-103``).
    The online (running-max) formulation of the kernel is algebraically this
    two-pass softmax.  ``causal=False`` drops the mask (every query sees all
    ``t_k`` keys), the unmasked case of the same kernel.
    """
    hd = q.shape[-1]
    t_q, t_k = q.shape[-2], k.shape[-2]
    scale = 1.0 / math.sqrt(hd)
    s = (q @ k.transpose(-1, -2)) * scale
    # query i sits at absolute position (t_k - t_q + i): the prefill case has
    # t_q == t_k; a decode step (t_q == 1) sees every cached key.
    qi = torch.arange(t_q).unsqueeze(1) + (t_k - t_q)
    kj = torch.arange(t_k).unsqueeze(0)
    if causal:
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
    return forward_cached(w, idx, n_head, flow)[0]


def forward_cached(w: Dict[str, torch.Tensor], idx: torch.Tensor, n_head: int,
                   flow: Flow = FLOWS["fp32"], cache: Optional[list] = None):
    """The forward of ``gpt_forward`` for tokens at positions p0 .. p0+T-1, where
    p0 is the number of positions already held in ``cache`` (a list of per-layer
    (k, v) tensors (B, H, p0, hd), stored in ``flow.act`` as the QKV projection
    rounds them; None or empty for p0 = 0).  Returns (logits (B, T, V), the
    cache extended by these T positions).

    Every op but attention is row-local, and attention of a query at position p
    reads only keys 0..p (``attention.py:90-94``), so running positions in two
    parts with the earlier keys and values kept equals running them together:
    this is the reference's full recompute (``models/gpt.py:204-206``) without
    recomputing the prefix.
    """
    c = flow.compute

    def W(key: str) -> torch.Tensor:
        return w[key].to(c)

    B, T = idx.shape
    D = w["wte"].shape[1]
    hd = D // n_head
    p0 = 0 if not cache else cache[0][0].shape[2]
    new_cache = []
    # gpt.py:110-113
    tok = embedding(idx, W("wte"))
    pos = embedding(torch.arange(p0, p0 + T), W("wpe"))
    x = round_to(tok + pos.unsqueeze(0), flow.resid)
    for i in range(_n_layer(w)):
        p = f"h.{i}."
        # gpt.py:120-137
        h = round_to(layer_norm(x, W(p + "ln_1.weight"), W(p + "ln_1.bias")), flow.act)
        qkv = round_to(linear(h, W(p + "attn.c_attn.weight"), W(p + "attn.c_attn.bias")), flow.act)
        q, k, v = qkv.split(D, dim=2)
        q, k, v = (t.reshape(B, T, n_head, hd).transpose(1, 2) for t in (q, k, v))
        if cache:
            k = torch.cat([cache[i][0], k], dim=2)
            v = torch.cat([cache[i][1], v], dim=2)
        new_cache.append((k, v))
        # gpt.py:140-155 (queries at positions p0.., keys 0..p0+T-1)
        if flow.online_lazy is None:
            a = causal_attention(q, k, v, flow.p)
        else:
            a = online_attention(q, k, v, flow.p, lazy_log2=flow.online_lazy)
        a = round_to(a, flow.act)
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
    return round_to(linear(h, W("lm_head.weight")), flow.logits), new_cache


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


@torch.inference_mode()
def generate_cached(w: Dict[str, torch.Tensor], idx: torch.Tensor, n_head: int,
                    max_new_tokens: int, flow: Flow = FLOWS["fp32"],
                    return_logits: bool = False):
    """``generate`` (greedy) with the keys and values of earlier positions kept
    (``forward_cached``) instead of re-running the whole prefix per token; the
    prompt plus new tokens must fit the context (no cropping).  With
    ``return_logits`` also returns the last-position logits of every step
    (B, max_new_tokens, V)."""
    out, seen = idx, []
    logits, cache = forward_cached(w, idx, n_head, flow)
    for t in range(max_new_tokens):
        last = logits[:, -1, :]
        seen.append(last)
        nxt = last.argmax(-1, keepdim=True)
        out = torch.cat([out, nxt], dim=1)
        if t + 1 < max_new_tokens:
            logits, cache = forward_cached(w, nxt, n_head, flow, cache)
    if return_logits:
        return out, torch.stack(seen, dim=1)
    return out


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


AFFINE_KEYS = ("ln_1.weight", "ln_1.bias", "attn.c_attn.bias", "attn.c_proj.bias",
               "ln_2.weight", "ln_2.bias", "mlp.c_fc.bias", "mlp.c_proj.bias")


def randomize_affine(w: Dict[str, torch.Tensor], seed: int, std: float = 0.1) -> Dict[str, torch.Tensor]:
    """A copy of ``w`` whose every bias and LayerNorm beta is ~N(0, std) and
    every LayerNorm gamma ~N(1, std), as a trained checkpoint has them (the
    reference's loader maps each of these tensors, ``models/gpt.py:266-296``,
    and the forward uses each at its own place, ``:120-177``).

    Every tensor is drawn separately, in the fixed order layer by layer over
    ``AFFINE_KEYS`` and then ``ln_f``, from ``torch.Generator().manual_seed(seed)``
    in fp32 and cast to the dtype it replaces, so two tensors of one shape
    differ and a swap of any two changes the forward.  Matrices, embeddings and
    a tied ``lm_head.weight`` are shared with ``w``."""
    g = torch.Generator().manual_seed(seed)
    out = dict(w)
    names = [f"h.{i}.{k}" for i in range(_n_layer(w)) for k in AFFINE_KEYS]
    for key in names + ["ln_f.weight", "ln_f.bias"]:
        ref = w[key]
        t = torch.randn(ref.shape, generator=g, dtype=torch.float32) * std
        if key.endswith(("ln_1.weight", "ln_2.weight", "ln_f.weight")):
            t = t + 1.0
        out[key] = t.to(ref.dtype)
    return out
