"""Drop-in replacements for cutileGPT's kernel functions, on torch tensors.

Each ``cutile_*`` function keeps the name, argument meaning and output shape of
the reference function it replaces (cited per function), runs one or more of
the hand-written gfx950 kernels of ``libcgpt.so`` on
``torch.cuda.current_stream()``, returns a freshly allocated output and never
mutates its inputs.  Tensors must live on the GPU; anything else raises
``ValueError`` (the reference raises ``ValueError`` for non-device arrays, e.g.
``cutile_gpt/kernels/gelu.py:81-82``).  Supported dtypes: float32, bfloat16 and
float16 (the reference's wrappers take float32 and float16).

The fused entry points (``add_layer_norm``, ``linear_bias_gelu``,
``attention_qkv``, ``token_pos_embedding``) are what ``CutileGPT.forward`` uses;
they remove the HBM round trips the reference spends on separate residual adds,
GELU passes and QKV split/transpose copies.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from .tiles import gemm_tile

_DT = {torch.float32: _lib.CGPT_F32, torch.bfloat16: _lib.CGPT_BF16,
       torch.float16: _lib.CGPT_F16}


def _dtype_code(t: torch.Tensor, name: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"{name}: unsupported dtype {t.dtype} "
                         "(float32, bfloat16 or float16)") from None


def _require_gpu(name: str, *tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"{name}: tensors must be torch tensors on the GPU")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous tensor whose data pointer is 16-byte aligned."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


# ---------------------------------------------------------------------------
# GELU


def cutile_gelu(x: torch.Tensor) -> torch.Tensor:
    """tanh-approximate GELU of any-shaped ``x``.

    Replaces ``cutile_gelu`` (``cutile_gpt/kernels/gelu.py:71-110``).
    """
    _require_gpu("cutile_gelu", x)
    code = _dtype_code(x, "cutile_gelu")
    xc = _aligned(x)
    y = torch.empty_like(xc)
    lib = _lib.load()
    _lib.check(lib.cgpt_gelu(xc.data_ptr(), y.data_ptr(), xc.numel(), code, _stream()),
               "cutile_gelu")
    return y.view(x.shape)


# ---------------------------------------------------------------------------
# LayerNorm (+ residual add)


def add_layer_norm(x: torch.Tensor, delta: Optional[torch.Tensor], weight: torch.Tensor,
                   bias: torch.Tensor, eps: float = 1e-5, out_dtype: Optional[torch.dtype] = None,
                   x_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``s = x + delta`` (delta optional); writes ``s`` into ``x_out`` when given
    (it may be ``x`` itself) and returns ``LayerNorm(s)`` in ``out_dtype``.

    One kernel for the residual adds at ``cutile_gpt/models/gpt.py:155,174`` and
    ``cutile_layer_norm`` (``cutile_gpt/kernels/layernorm.py:77-135``).
    """
    _require_gpu("add_layer_norm", x, delta, weight, bias, x_out)
    n = x.shape[-1]
    if weight.numel() != n or bias.numel() != n:
        raise ValueError(f"add_layer_norm: weight/bias must have {n} elements")
    if delta is not None and delta.shape != x.shape:
        raise ValueError("add_layer_norm: delta must have the shape of x")
    if x_out is not None and (x_out.shape != x.shape or x_out.dtype != x.dtype
                              or not x_out.is_contiguous()):
        raise ValueError("add_layer_norm: x_out must be a contiguous tensor like x")
    xc = x if x.is_contiguous() else x.contiguous()
    dc = None if delta is None else (delta if delta.is_contiguous() else delta.contiguous())
    w = weight.contiguous()
    b = bias.contiguous()
    if b.dtype != w.dtype:
        b = b.to(w.dtype)
    out_dtype = out_dtype or x.dtype
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    lib = _lib.load()
    rows = xc.numel() // n if n else 0
    _lib.check(lib.cgpt_add_layernorm(
        xc.data_ptr(), None if dc is None else dc.data_ptr(),
        None if x_out is None else x_out.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(),
        rows, n, float(eps), _dtype_code(xc, "x"),
        _dtype_code(dc, "delta") if dc is not None else 0, _dtype_code(w, "weight"),
        _dtype_code(y, "out"), _stream()), "add_layer_norm")
    return y


def cutile_layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                      eps: float = 1e-5) -> torch.Tensor:
    """LayerNorm over the last axis (biased variance), output in ``x.dtype``.

    Replaces ``cutile_layer_norm`` (``cutile_gpt/kernels/layernorm.py:77-135``)
    for rows of any width, without the reference's power-of-two padding copies:
    rows of a multiple of 4 up to 4096 elements stay in registers (float32,
    bfloat16, or float16 throughout), other widths and dtype mixes take a
    block-per-row kernel.
    """
    return add_layer_norm(x, None, weight, bias, eps)


# ---------------------------------------------------------------------------
# Linear / GEMM


def _gemm(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], epilogue: int,
          out_dtype: Optional[torch.dtype], name: str, out: Optional[torch.Tensor] = None,
          tile: Optional[int] = None) -> torch.Tensor:
    _require_gpu(name, x, weight, bias)
    k = x.shape[-1]
    if weight.dim() != 2 or weight.shape[1] != k:
        raise ValueError(f"{name}: weight must be (out_features, {k}), got {tuple(weight.shape)}")
    if weight.dtype != x.dtype:
        raise ValueError(f"{name}: x and weight dtypes differ ({x.dtype} vs {weight.dtype})")
    n = weight.shape[0]
    if bias is not None and bias.numel() != n:
        raise ValueError(f"{name}: bias must have {n} elements")
    a = _aligned(x.reshape(-1, k))
    w = weight if (weight.stride(1) == 1 and weight.stride(0) % 8 == 0
                   and weight.data_ptr() % 16 == 0) else _aligned(weight)
    m = a.shape[0]
    out_dtype = out_dtype or x.dtype
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    b = None if bias is None else _aligned(bias)
    lib = _lib.load()
    in_code = _dtype_code(a, name)
    t = gemm_tile(in_code, m, n, k) if tile is None else tile
    _lib.check(lib.cgpt_gemm(
        a.data_ptr(), w.data_ptr(), None if b is None else b.data_ptr(), out.data_ptr(),
        m, n, k, a.stride(0), w.stride(0), out.stride(0), in_code,
        _dtype_code(b, "bias") if b is not None else 0, _dtype_code(out, "out"), epilogue, t,
        _stream()), name)
    return out.view(*x.shape[:-1], n)


def cutile_linear(x: torch.Tensor, weight: torch.Tensor,
                  weight_t: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``y = x @ weight.T`` with ``weight`` (out_features, in_features).

    Replaces ``cutile_linear`` (``cutile_gpt/kernels/linear.py:112-161``).  The
    kernel consumes ``weight`` in its own (out, in) layout, so ``weight_t`` (the
    reference's pre-transposed copy) is accepted for compatibility and unused.
    """
    return _gemm(x, weight, None, _lib.EPI_NONE, None, "cutile_linear")


def cutile_linear_bias(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                       weight_t: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``y = x @ weight.T + bias``.

    Replaces ``cutile_linear_bias`` (``cutile_gpt/kernels/linear.py:164-222``).
    """
    return _gemm(x, weight, bias, _lib.EPI_BIAS, None, "cutile_linear_bias")


def linear_bias_gelu(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """``gelu_tanh(x @ weight.T + bias)`` with GELU applied in the GEMM epilogue
    (``cutile_gpt/models/gpt.py:161-167`` in one kernel)."""
    return _gemm(x, weight, bias, _lib.EPI_BIAS_GELU, None, "linear_bias_gelu")


def cutile_fused_mlp(x: torch.Tensor, w_fc: torch.Tensor, b_fc: torch.Tensor,
                     w_proj: torch.Tensor, b_proj: torch.Tensor) -> torch.Tensor:
    """``gelu(x W_fc^T + b_fc) W_proj^T + b_proj``.

    Same result as ``cutile_fused_mlp`` (``cutile_gpt/kernels/fused_mlp.py:112-161``),
    composed from the up-projection GEMM with the GELU epilogue and the
    down-projection GEMM instead of one kernel that recomputes the hidden strip
    per output tile.
    """
    return cutile_linear_bias(linear_bias_gelu(x, w_fc, b_fc), w_proj, b_proj)


# ---------------------------------------------------------------------------
# Attention


def _attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, B: int, H: int,
               Tq: int, Tk: int, hd: int, qs, ks, vs, os_, scale: float, causal: bool,
               name: str) -> None:
    lib = _lib.load()
    _lib.check(lib.cgpt_attention_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Tq, Tk, hd,
        *qs, *ks, *vs, *os_, float(scale), int(causal), _dtype_code(q, name), _stream()), name)


_ATTN_HD = (16, 32, 64, 128)  # head_dim values the attention kernels are built for


def cutile_causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            n_head: int) -> torch.Tensor:
    """Causal softmax attention on (batch, n_head, seq_len, head_dim) tensors.

    Replaces ``cutile_causal_attention`` (``cutile_gpt/kernels/attention.py:119-175``).
    Inputs may be any strided views whose last axis is contiguous (no copies);
    the output is a new contiguous tensor.  The kernels take head_dim 16, 32, 64
    or 128; other head_dim up to 128 are zero-padded to the next of those (the
    padded columns add 0 to every score and give output columns that are
    dropped; the scale stays 1/sqrt(head_dim)).
    """
    _require_gpu("cutile_causal_attention", q, k, v)
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("cutile_causal_attention: q, k, v must share shape (B, H, T, hd)")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("cutile_causal_attention: q, k, v dtypes differ")
    B, H, T, hd = q.shape
    hp = next((d for d in _ATTN_HD if d >= hd), None)
    if hd < 1 or hp is None:
        raise ValueError(f"cutile_causal_attention: head_dim {hd} outside 1..{_ATTN_HD[-1]}")
    if hp != hd:
        pad = lambda t: torch.nn.functional.pad(t, (0, hp - hd))
        o = torch.empty((B, H, T, hp), dtype=q.dtype, device=q.device)
        qp, kp, vp = pad(q), pad(k), pad(v)
        _attention(qp, kp, vp, o, B, H, T, T, hp, qp.stride()[:3], kp.stride()[:3],
                   vp.stride()[:3], o.stride()[:3], 1.0 / math.sqrt(hd), True,
                   "cutile_causal_attention")
        return o[..., :hd].contiguous()

    def fix(t):
        if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]):
            t = t.contiguous()
        return t

    q, k, v = fix(q), fix(k), fix(v)
    o = torch.empty((B, H, T, hd), dtype=q.dtype, device=q.device)
    _attention(q, k, v, o, B, H, T, T, hd, q.stride()[:3], k.stride()[:3], v.stride()[:3],
               o.stride()[:3], 1.0 / math.sqrt(hd), True, "cutile_causal_attention")
    return o


def attention_qkv(qkv: torch.Tensor, n_head: int, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention straight from the fused projection buffer.

    ``qkv`` is (B, T, 3*D) as produced by the c_attn GEMM; the result is (B, T, D)
    with heads interleaved, ready for c_proj.  Replaces the split / reshape /
    transpose / ``ascontiguousarray`` glue around attention at
    ``cutile_gpt/models/gpt.py:133-146`` with strided addressing in the kernel.
    """
    name = "attention_qkv"
    _require_gpu(name, qkv, out)
    _dtype_code(qkv, name)
    if qkv.dim() != 3 or qkv.shape[2] % 3:
        raise ValueError(f"{name}: qkv must be (B, T, 3*D), got {tuple(qkv.shape)}")
    B, T, D3 = qkv.shape
    D = D3 // 3
    if n_head <= 0 or D % n_head:
        raise ValueError(f"{name}: D={D} is not divisible by n_head={n_head}")
    hd = D // n_head
    # Strides come from the tensor itself (a view such as qkv[:, :T2] keeps its
    # parent's batch stride); the element axis must be contiguous.
    sb, st_, se = qkv.stride()
    if se != 1:
        raise ValueError(f"{name}: the last axis of qkv must be contiguous")
    if out is None:
        out = torch.empty((B, T, D), dtype=qkv.dtype, device=qkv.device)
    elif out.shape != (B, T, D) or out.dtype != qkv.dtype or not out.is_contiguous():
        raise ValueError(f"{name}: out must be a contiguous {qkv.dtype} tensor of shape "
                         f"{(B, T, D)}, got {out.dtype} {tuple(out.shape)}")
    elif out.device != qkv.device:
        raise ValueError(f"{name}: out is on {out.device}, qkv on {qkv.device}")
    st = (sb, hd, st_)
    q = qkv
    k = qkv[..., D:]
    v = qkv[..., 2 * D:]
    _attention(q, k, v, out, B, n_head, T, T, hd, st, st, st, (T * D, hd, D),
               1.0 / math.sqrt(hd), True, name)
    return out


# ---------------------------------------------------------------------------
# Embedding


def token_pos_embedding(idx: torch.Tensor, wte: torch.Tensor, wpe: Optional[torch.Tensor],
                        pos0: int = 0, out_dtype: Optional[torch.dtype] = None,
                        err_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``wte[idx] + wpe[pos0 + t]`` for ``idx`` (B, T) -> (B, T, D).

    Replaces ``cutile_embedding`` twice plus the broadcast add at
    ``cutile_gpt/models/gpt.py:110-113`` with one gather kernel.
    """
    _require_gpu("token_pos_embedding", idx, wte, wpe)
    idx64 = idx if idx.dtype == torch.int64 and idx.is_contiguous() else idx.to(torch.int64).contiguous()
    D = wte.shape[1]
    T = idx.shape[-1] if idx.dim() else 1
    out = torch.empty((*idx.shape, D), dtype=out_dtype or wte.dtype, device=wte.device)
    w = wte.contiguous()
    p = None if wpe is None else wpe.contiguous()
    lib = _lib.load()
    _lib.check(lib.cgpt_embedding(
        idx64.data_ptr(), w.data_ptr(), None if p is None else p.data_ptr(), out.data_ptr(),
        idx64.numel(), max(T, 1), D, w.shape[0], pos0, 0 if p is None else p.shape[0],
        _dtype_code(w, "wte"), _dtype_code(out, "out"),
        None if err_flag is None else err_flag.data_ptr(), _stream()), "token_pos_embedding")
    return out


def cutile_embedding(indices: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Row gather ``weight[indices]`` -> (*indices.shape, n_embd).

    Replaces ``cutile_embedding`` (``cutile_gpt/kernels/embedding.py:54-109``)
    without the reference's padded copy of the whole table.  Ids outside
    [0, vocab) raise ``IndexError`` (checked on the host after the launch).
    """
    _require_gpu("cutile_embedding", indices, weight)
    flag = torch.zeros(1, dtype=torch.int32, device=weight.device)
    idx = indices.reshape(-1)
    out = token_pos_embedding(idx.view(1, -1), weight, None, err_flag=flag)
    if int(flag.item()) != 0:
        raise IndexError("cutile_embedding: index out of range of the embedding table")
    return out.view(*indices.shape, weight.shape[1])
