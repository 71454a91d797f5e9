"""CutileGPT: the reference's model API on the gfx950 kernels of libcgpt.so.

Same surface as ``cutile_gpt/models/gpt.py:24-343``: ``CutileGPT(config)``, the
``weights`` dict with the reference's keys and (out, in) Linear layout,
``forward(idx) -> (logits, None)`` / ``__call__``, ``generate``,
``load_from_huggingface`` (local HF directory) and ``load_from_mingpt``.

Forward data flow on one GPU (M = B*T rows, D = n_embd):

    x  (M, D)  fp32 residual stream           <- embedding gather + position add,
    h  (M, D)  act dtype  = LN1(x)                fused with layer 0's LayerNorm
    qkv(M, 3D) act dtype  = h Wqkv^T + b       <- MFMA GEMM, bias epilogue
    a  (M, D)  act dtype  = attention(qkv)     <- flash attention reading qkv strided
    x += a Wo^T + b                            <- GEMM with the residual add in its
                                                  epilogue (fp32: the residual stream
                                                  never takes a rounded delta)
    h = LN2(x)                                 <- LayerNorm
    f  (M, 4D) act dtype  = gelu(h Wfc^T + b)  <- GEMM with GELU epilogue
    x += f Wp^T + b                            <- GEMM with the residual add
    h = LN1'(x) (next layer, or ln_f)          <- LayerNorm
    logits (M, V) fp32    = h wte^T            <- GEMM (tied head, no bias)

``act dtype`` is the model dtype (float32 or bfloat16).  There is no CPU or
PyTorch fallback: without libcgpt.so the forward raises.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

from . import _lib
from .config import GPTConfig
from .tiles import gemm_tile

_DT = {torch.float32: _lib.CGPT_F32, torch.bfloat16: _lib.CGPT_BF16}


class CutileGPT:
    """GPT-2 inference model (pre-LN, tanh-GELU, tied embeddings)."""

    def __init__(self, config: GPTConfig, dtype: torch.dtype = torch.float32,
                 device: str = "cuda", seed: Optional[int] = None,
                 logits_dtype: torch.dtype = torch.float32, init_weights: bool = True):
        if dtype not in _DT:
            raise ValueError(f"dtype must be float32 or bfloat16, got {dtype}")
        if config.n_embd % config.n_head:
            raise ValueError("n_embd must be divisible by n_head")
        self.config = config
        self.dtype = dtype
        self.device = torch.device(device)
        self.logits_dtype = logits_dtype
        self.weights: Dict[str, torch.Tensor] = {}
        self._err = None
        self._decode_session = None  # the last generate()'s KV cache and step graphs
        if init_weights:
            self._init_weights(seed)

    # ------------------------------------------------------------------ weights

    def _init_weights(self, seed: Optional[int] = None) -> None:
        """Random init as ``cutile_gpt/models/gpt.py:39-81`` (seeded when ``seed``
        is given): wte, wpe, c_attn, c_fc ~ N(0, 0.02); both c_proj ~
        N(0, 0.02/sqrt(2 n_layer)); LN weight 1, biases 0; lm_head tied to wte."""
        cfg = self.config
        g = torch.Generator().manual_seed(seed) if seed is not None else None
        D = cfg.n_embd
        proj = 0.02 / math.sqrt(2 * cfg.n_layer)

        def randn(*shape, std=0.02):
            return torch.randn(*shape, generator=g) * std

        w = {"wte": randn(cfg.vocab_size, D), "wpe": randn(cfg.block_size, D)}
        for i in range(cfg.n_layer):
            p = f"h.{i}."
            w[p + "ln_1.weight"] = torch.ones(D)
            w[p + "ln_1.bias"] = torch.zeros(D)
            w[p + "attn.c_attn.weight"] = randn(3 * D, D)
            w[p + "attn.c_attn.bias"] = torch.zeros(3 * D)
            w[p + "attn.c_proj.weight"] = randn(D, D, std=proj)
            w[p + "attn.c_proj.bias"] = torch.zeros(D)
            w[p + "ln_2.weight"] = torch.ones(D)
            w[p + "ln_2.bias"] = torch.zeros(D)
            w[p + "mlp.c_fc.weight"] = randn(4 * D, D)
            w[p + "mlp.c_fc.bias"] = torch.zeros(4 * D)
            w[p + "mlp.c_proj.weight"] = randn(D, 4 * D, std=proj)
            w[p + "mlp.c_proj.bias"] = torch.zeros(D)
        w["ln_f.weight"] = torch.ones(D)
        w["ln_f.bias"] = torch.zeros(D)
        self.load_weights(w)

    def load_weights(self, weights: Dict[str, torch.Tensor]) -> None:
        """Install a weight dict in the reference's key layout (Linear weights
        (out, in)); tensors are copied to the model's device and dtype as
        contiguous, 16-byte aligned buffers.  ``lm_head.weight`` defaults to
        (and, when equal to it, shares storage with) ``wte``."""
        cfg = self.config
        self._decode_session = None
        out: Dict[str, torch.Tensor] = {}
        for k, v in weights.items():
            if k == "lm_head.weight":
                continue
            t = v.detach().to(device=self.device, dtype=self.dtype).contiguous()
            if t.data_ptr() % 16:
                t = t.clone()
            out[k] = t
        head = weights.get("lm_head.weight")
        if head is None or head is weights.get("wte") or (
                head.shape == weights["wte"].shape and head.data_ptr() == weights["wte"].data_ptr()):
            out["lm_head.weight"] = out["wte"]
        else:
            out["lm_head.weight"] = head.detach().to(device=self.device, dtype=self.dtype).contiguous()
        expect = {"wte": (cfg.vocab_size, cfg.n_embd), "wpe": (cfg.block_size, cfg.n_embd)}
        for k, shp in expect.items():
            if tuple(out[k].shape) != shp:
                raise ValueError(f"{k} has shape {tuple(out[k].shape)}, expected {shp}")
        # The LM head's B operand padded with zero rows to a multiple of 64
        # (50257 -> 50304): the head GEMM then has N % 64 == 0, every output
        # row is 16-byte aligned (vector and buffer-resource stores) and the
        # 256x192 tiles cover it exactly.  wte (and a tied lm_head) are views
        # of the first vocab_size rows, so nothing is duplicated.
        V, D = cfg.vocab_size, cfg.n_embd
        vp = (V + 63) // 64 * 64
        tied = out["lm_head.weight"] is out["wte"]
        if vp == V:
            self._head_pad = out["lm_head.weight"]
        else:
            pad = torch.zeros((vp, D), dtype=self.dtype, device=self.device)
            pad[:V].copy_(out["lm_head.weight"])
            self._head_pad = pad
            if tied:
                out["wte"] = pad[:V]
                out["lm_head.weight"] = out["wte"]
            else:
                out["lm_head.weight"] = pad[:V]
        self.weights = out

    @property
    def weight_transposes(self) -> Dict[str, torch.Tensor]:
        """(in, out) views of every 2-D weight (the reference caches copies,
        ``models/gpt.py:83-90``; the GEMM here reads (out, in) directly)."""
        return {k: v.t() for k, v in self.weights.items() if "weight" in k and v.dim() == 2}

    # ------------------------------------------------------------------ forward

    def __call__(self, idx: torch.Tensor) -> Tuple[torch.Tensor, None]:
        return self.forward(idx)

    def _prepare_idx(self, idx: torch.Tensor) -> torch.Tensor:
        if idx.dim() != 2:
            raise ValueError(f"idx must be (batch, seq_len), got {tuple(idx.shape)}")
        if not idx.is_cuda:
            if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= self.config.vocab_size):
                raise IndexError("token id out of range of the vocabulary")
            idx = idx.to(self.device, non_blocking=True)
        if idx.dtype != torch.int64 or not idx.is_contiguous():
            idx = idx.to(torch.int64).contiguous()
        return idx

    @torch.inference_mode()
    def forward(self, idx: torch.Tensor, probe=None) -> Tuple[torch.Tensor, None]:
        """Logits (B, T, vocab) for token ids ``idx`` (B, T); restates
        ``cutile_gpt/models/gpt.py:95-183`` on the fused kernels.

        ``probe``, when given, is called as ``probe(tag, True)`` right before and
        ``probe(tag, False)`` right after each kernel launch (tags: embedding,
        ln, gemm_qkv, attention, gemm_proj, gemm_fc_gelu, gemm_mlp_proj,
        lm_head) — a hook for timing individual launches with stream events."""
        return self._forward(idx, probe=probe), None

    def _forward(self, idx: torch.Tensor, probe=None, cache=None,
                 logits_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Forward body.  ``cache`` (a ``decode.KVCache``): also store every
        layer's keys and values at positions 0..T-1.  ``logits_out`` (B, vocab):
        compute the LM head for the last position of each sequence only, into
        that tensor, and return it."""
        B, T = idx.shape
        cfg = self.config
        assert T <= cfg.block_size, f"Sequence length {T} > block_size {cfg.block_size}"
        idx = self._prepare_idx(idx)
        lib = _lib.load()
        chk = _lib.check
        W = self.weights
        D, H, V = cfg.n_embd, cfg.n_head, cfg.vocab_size
        hd = D // H
        M = B * T
        dev = self.device
        act = self.dtype
        ac = _DT[act]
        f32 = _lib.CGPT_F32
        s = torch.cuda.current_stream(dev).cuda_stream
        if self._err is None:
            self._err = torch.zeros(1, dtype=torch.int32, device=dev)

        x = torch.empty((M, D), dtype=torch.float32, device=dev)
        h = torch.empty((M, D), dtype=act, device=dev)
        qkv = torch.empty((M, 3 * D), dtype=act, device=dev)
        att = torch.empty((M, D), dtype=act, device=dev)
        f = torch.empty((M, 4 * D), dtype=act, device=dev)
        Vp = self._head_pad.shape[0]
        logits = (torch.empty((M, Vp), dtype=self.logits_dtype, device=dev)
                  if logits_out is None else None)
        px, ph, pq, pa, pf = (t.data_ptr() for t in (x, h, qkv, att, f))

        mark = probe if probe is not None else (lambda tag, start: None)

        def gemm(tag, a_ptr, w, b, c_ptr, n, k, epi, out_code):
            t = gemm_tile(ac, M, n, k)
            mark(tag, True)
            chk(lib.cgpt_gemm(a_ptr, w.data_ptr(), None if b is None else b.data_ptr(), c_ptr,
                              M, n, k, k, w.stride(0), n, ac, ac, out_code, epi, t, s), tag)
            mark(tag, False)

        def ln(wk):
            # h = LayerNorm(x); x itself is left as it is.
            mark("ln", True)
            chk(lib.cgpt_add_layernorm(px, None, None, W[wk + ".weight"].data_ptr(),
                                       W[wk + ".bias"].data_ptr(), ph, M, D, 1e-5, f32, f32, ac,
                                       ac, s), "layernorm")
            mark("ln", False)

        # x = wte[idx] + wpe[pos] and h = ln_1(x) of layer 0 in one pass.
        mark("embedding", True)
        chk(lib.cgpt_embedding_layernorm(idx.data_ptr(), W["wte"].data_ptr(), W["wpe"].data_ptr(),
                                         None, px, W["h.0.ln_1.weight"].data_ptr(),
                                         W["h.0.ln_1.bias"].data_ptr(), ph, M, T, D, V, 0,
                                         cfg.block_size, 1e-5, ac, ac, self._err.data_ptr(), s),
            "embedding_layernorm")
        mark("embedding", False)
        st_qkv = (T * 3 * D, hd, 3 * D)
        st_o = (T * D, hd, D)
        scale = 1.0 / math.sqrt(hd)
        for i in range(cfg.n_layer):
            p = f"h.{i}."
            gemm("gemm_qkv", ph, W[p + "attn.c_attn.weight"], W[p + "attn.c_attn.bias"], pq,
                 3 * D, D, _lib.EPI_BIAS, ac)
            esz = qkv.element_size()
            if cache is not None:
                csb, csh, cst = cache.strides()
                chk(lib.cgpt_kv_store(pq + D * esz, pq + 2 * D * esz, cache.k[i].data_ptr(),
                                      cache.v[i].data_ptr(), B, H, T, hd, 0, cache.t_max,
                                      *st_qkv, *st_qkv, csb, csh, cst, ac, s), "kv_store")
            mark("attention", True)
            chk(lib.cgpt_attention_fwd(pq, pq + D * esz, pq + 2 * D * esz, pa, B, H, T, T, hd,
                                       *st_qkv, *st_qkv, *st_qkv, *st_o, scale, 1, ac, s),
                "attention")
            mark("attention", False)
            # x += att Wo^T + b (residual add in the GEMM epilogue, in place)
            gemm("gemm_proj", pa, W[p + "attn.c_proj.weight"], W[p + "attn.c_proj.bias"], px,
                 D, D, _lib.EPI_BIAS_RESID, f32)
            ln(p + "ln_2")
            gemm("gemm_fc_gelu", ph, W[p + "mlp.c_fc.weight"], W[p + "mlp.c_fc.bias"], pf,
                 4 * D, D, _lib.EPI_BIAS_GELU, ac)
            gemm("gemm_mlp_proj", pf, W[p + "mlp.c_proj.weight"], W[p + "mlp.c_proj.bias"], px,
                 D, 4 * D, _lib.EPI_BIAS_RESID, f32)
            ln("ln_f" if i + 1 == cfg.n_layer else f"h.{i + 1}.ln_1")
        if logits_out is not None:
            # Last position of each sequence: rows b*T + T-1 of h, stride T*D.
            mark("lm_head", True)
            chk(lib.cgpt_gemm(ph + (T - 1) * D * h.element_size(), W["lm_head.weight"].data_ptr(),
                              None, logits_out.data_ptr(), B, V, D, T * D,
                              W["lm_head.weight"].stride(0), V, ac, ac, _DT[logits_out.dtype],
                              _lib.EPI_NONE, _lib.TILE_AUTO, s), "lm_head")
            mark("lm_head", False)
            return logits_out
        # Padded head: logits rows have stride Vp; the returned (B, T, V) tensor
        # is a view of the first V columns.
        mark("lm_head", True)
        head = self._head_pad
        chk(lib.cgpt_gemm(ph, head.data_ptr(), None, logits.data_ptr(), M, Vp, D, D, head.stride(0),
                          Vp, ac, ac, _DT[self.logits_dtype], _lib.EPI_NONE,
                          gemm_tile(ac, M, Vp, D), s), "lm_head")
        mark("lm_head", False)
        return logits[:, :V].view(B, T, V)

    def input_errors(self) -> bool:
        """True if any forward so far saw a token id outside the vocabulary
        (such ids are clamped by the gather kernel).  Synchronises."""
        return self._err is not None and int(self._err.item()) != 0

    # --------------------------------------------------------------- generation

    @torch.inference_mode()
    def generate(self, idx: torch.Tensor, max_new_tokens: int, temperature: float = 1.0,
                 top_k: Optional[int] = None, use_cache: bool = True,
                 use_graph: bool = True) -> torch.Tensor:
        """Autoregressive continuation with the semantics of
        ``cutile_gpt/models/gpt.py:185-229``: temperature, top-k masking, then
        sampling; ``top_k=1`` is greedy decoding.

        With ``use_cache`` (and prompt + new tokens within block_size, at most
        64 sequences) the prompt is run once and each new token costs one
        KV-cache step (``decode.DecodeSession``); greedy steps run entirely on
        the device and are replayed from one captured HIP graph when
        ``use_graph``.  Otherwise every token re-runs the full forward on the
        last block_size tokens, as the reference does."""
        idx = self._prepare_idx(idx)
        B, T0 = idx.shape
        if max_new_tokens <= 0:
            return idx
        if use_cache and T0 + max_new_tokens <= self.config.block_size and B <= 64:
            from .decode import DecodeSession

            # The last session (its cache, buffers and captured step graphs)
            # serves the next call of the same shape while the model holds
            # the same weight tensors.
            sess = self._decode_session
            if sess is None or not sess.matches(B, T0, max_new_tokens):
                self._decode_session = None
                sess = DecodeSession(self, B, T0, max_new_tokens)
                self._decode_session = sess
            sess.prefill(idx)
            if top_k == 1:
                new = sess.run_greedy(use_graph=use_graph)
                return torch.cat([idx, new], dim=1)
            sess.step.zero_()
            sess.err.zero_()
            out = []
            for t in range(max_new_tokens):
                if t > 0:
                    sess.next_logits(use_graph=use_graph and max_new_tokens >= 4)
                nxt = self._sample(sess.logits, temperature, top_k)
                out.append(nxt)
                sess.ids.copy_(nxt.view(-1))
                if t > 0:
                    sess.step.add_(1)
            return torch.cat([idx] + out, dim=1)
        for _ in range(max_new_tokens):
            cond = idx if idx.shape[1] <= self.config.block_size else idx[:, -self.config.block_size:]
            logits = self._forward(cond)
            nxt = self._sample(logits[:, -1, :], temperature, top_k)
            idx = torch.cat([idx, nxt], dim=1)
        return idx

    @staticmethod
    def _sample(logits: torch.Tensor, temperature: float, top_k: Optional[int]) -> torch.Tensor:
        """Next token (B, 1) from last-position logits (B, V): temperature,
        top-k masking, argmax for top_k == 1 else multinomial sampling
        (``cutile_gpt/models/gpt.py:207-226``)."""
        logits = logits.float() / temperature
        if top_k is not None:
            k = min(top_k, logits.shape[-1])
            kth = torch.topk(logits, k, dim=-1).values[:, -1:]
            logits = logits.masked_fill(logits < kth, float("-inf"))
        if top_k == 1:
            return logits.argmax(-1, keepdim=True)
        probs = torch.softmax(logits, dim=-1)
        return torch.multinomial(probs, 1)

    # ------------------------------------------------------------------ loaders

    def load_from_huggingface(self, model_name: str = "gpt2") -> None:
        """Load GPT-2 weights from a local HF directory (``config.json`` +
        ``model.safetensors``) or, for a bare name, through transformers' cache.
        Mirrors ``cutile_gpt/models/gpt.py:231-304`` (Conv1D transposed, tied head)."""
        from .hf_loader import resolve_checkpoint

        w, config = resolve_checkpoint(model_name, device=str(self.device))
        for f in ("n_layer", "n_head", "n_embd", "vocab_size"):
            if getattr(config, f) != getattr(self.config, f):
                raise ValueError(f"checkpoint {f}={getattr(config, f)} does not match "
                                 f"model {f}={getattr(self.config, f)}")
        if config.block_size != self.config.block_size:
            raise ValueError("checkpoint n_positions does not match block_size")
        self.load_weights(w)

    def load_from_mingpt(self, mingpt_model) -> None:
        """Copy a minGPT model's weights (``cutile_gpt/models/gpt.py:306-343``):
        nn.Linear weights are already (out, in); ``lm_head.weight`` is kept as is."""
        sd = mingpt_model.state_dict()
        w = {"wte": sd["transformer.wte.weight"], "wpe": sd["transformer.wpe.weight"]}
        for i in range(self.config.n_layer):
            for name in ("ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias",
                         "attn.c_proj.weight", "attn.c_proj.bias", "ln_2.weight", "ln_2.bias",
                         "mlp.c_fc.weight", "mlp.c_fc.bias", "mlp.c_proj.weight",
                         "mlp.c_proj.bias"):
                w[f"h.{i}.{name}"] = sd[f"transformer.h.{i}.{name}"]
        w["ln_f.weight"] = sd["transformer.ln_f.weight"]
        w["ln_f.bias"] = sd["transformer.ln_f.bias"]
        w["lm_head.weight"] = sd["lm_head.weight"]
        self.load_weights(w)

    @classmethod
    def from_pretrained(cls, path: str, dtype: torch.dtype = torch.float32,
                        device: str = "cuda") -> "CutileGPT":
        """Build a model sized from an HF directory's config.json and load it."""
        from .hf_loader import resolve_checkpoint

        w, config = resolve_checkpoint(path, device=device)
        model = cls.__new__(cls)
        model.config = config
        model.dtype = dtype
        model.device = torch.device(device)
        model.logits_dtype = torch.float32
        model._err = None
        model.load_weights(w)
        return model
