"""KV-cache incremental decoding for CutileGPT (greedy or sampled).

The reference's ``generate`` (``cutile_gpt/models/gpt.py:185-229``) re-runs the
whole forward on the growing prefix for every new token.  Here a prompt is run
once (prefill) while its keys and values are stored into a per-layer cache,
and every further token costs one step over B rows:

    embedding at position pos        cgpt_embedding_layernorm (pos read on
      + LN_1 of layer 0                device, one pass)
    per layer: QKV GEMM              cgpt_gemm_partials (split-K partial products)
               attention             cgpt_attention_decode_partials (adds the
                                     partials + bias, appends k, v at pos)
               proj GEMM             cgpt_gemm_partials
               residual + LN_2       cgpt_add_layernorm_partials
               fc GEMM               cgpt_gemm_partials
               bias + GELU           cgpt_partials_bias_act (adds the partials)
               MLP proj GEMM         cgpt_gemm_partials
               residual + next LN    cgpt_add_layernorm_partials (LN_f last)
    LM head                          cgpt_gemm (skinny, N = vocab)
    greedy token                     cgpt_argmax (also written to the history)

The split-K GEMMs leave their K chunks' sums to the kernel that reads their
output, so a weight-streaming GEMM is one memory round trip with no
cross-block reduction; ``partials=False`` runs the earlier sequence instead
(bias GEMMs with an in-kernel split-K fix-up, separate residual+LN).

Everything a step reads or writes lives in buffers allocated once per
``generate`` call and the position is a device counter, so the greedy step is
captured once as a HIP graph and replayed for every token.

Cache layout, per layer: k and v of shape (B, H, t_max, head_dim) in the model
dtype, t_max = prompt length + new tokens (<= block_size).
"""

from __future__ import annotations

import ctypes
import gc
import math
import weakref
from typing import Optional

import torch

from . import _lib

_DT = {torch.float32: _lib.CGPT_F32, torch.bfloat16: _lib.CGPT_BF16}


class KVCache:
    """Keys and values of every layer: ``k[i]``, ``v[i]`` of shape (B, H, t_max, hd)."""

    def __init__(self, n_layer: int, B: int, H: int, t_max: int, hd: int, dtype: torch.dtype,
                 device: torch.device):
        self.t_max = t_max
        self.k = torch.empty((n_layer, B, H, t_max, hd), dtype=dtype, device=device)
        self.v = torch.empty((n_layer, B, H, t_max, hd), dtype=dtype, device=device)

    def strides(self):
        """(batch, head, time) element strides of one layer's k or v."""
        s = self.k[0].stride()
        return s[0], s[1], s[2]


class DecodeSession:
    """Buffers, cache and device counters of one batched generation."""

    def __init__(self, model, B: int, t0: int, max_new: int, partials: bool = True):
        # Ordinary (not inference-mode) tensors even when created inside
        # generate(): the session and its graphs outlive the call.
        with torch.inference_mode(False):
            self._init(model, B, t0, max_new, partials)

    def _init(self, model, B: int, t0: int, max_new: int, partials: bool) -> None:
        cfg = model.config
        if t0 + max_new > cfg.block_size:
            raise ValueError(f"prompt {t0} + {max_new} new tokens exceeds block_size {cfg.block_size}")
        if B > 64:
            raise ValueError("KV-cache decoding supports at most 64 sequences per batch")
        # A weak reference: the model keeps its last session (generate()), and
        # a model <-> session cycle would leave dead sessions, with their HIP
        # graphs, to the cyclic garbage collector, which may run inside a later
        # stream capture, where destroying a graph is an error.
        self._model = weakref.ref(model)
        self.B, self.t0, self.max_new = B, t0, max_new
        dev, act = model.device, model.dtype
        D, H, V = cfg.n_embd, cfg.n_head, cfg.vocab_size
        self.hd = D // H
        self.cache = KVCache(cfg.n_layer, B, H, t0 + max_new, self.hd, act, dev)
        self.ids = torch.zeros(B, dtype=torch.int64, device=dev)
        self.step = torch.zeros(1, dtype=torch.int32, device=dev)
        self.hist = torch.zeros((B, max_new), dtype=torch.int64, device=dev)
        self.x = torch.empty((B, D), dtype=torch.float32, device=dev)
        self.h = torch.empty((B, D), dtype=act, device=dev)
        self.qkv = torch.empty((B, 3 * D), dtype=act, device=dev)
        self.att = torch.empty((B, D), dtype=act, device=dev)
        self.delta = torch.empty((B, D), dtype=torch.float32, device=dev)
        self.f = torch.empty((B, 4 * D), dtype=act, device=dev)
        self.logits = torch.empty((B, V), dtype=model.logits_dtype, device=dev)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        # Captured greedy step and logits step, and the weight tensors they
        # were captured over (a graph holds device pointers).
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.graph_logits: Optional[torch.cuda.CUDAGraph] = None
        self._captured_over = None
        lib = _lib.load()
        # Split-K partial products of the QKV, attention-projection and
        # MLP-projection GEMMs, added by the attention and residual+LayerNorm
        # kernels that consume them (one buffer: the GEMMs run one after
        # another on one stream).
        self.partials = partials
        self.splits = {}
        p_max = 4
        for n, k in ((3 * D, D), (D, D), (4 * D, D), (D, 4 * D)):
            ns = ctypes.c_int64()
            _lib.check(lib.cgpt_gemm_partials_plan(B, n, k, _DT[act], ctypes.byref(ns)), "partials plan")
            self.splits[(n, k)] = ns.value
            p_max = max(p_max, ns.value * B * n)
        self.parts = torch.empty(p_max if partials else 4, dtype=torch.float32, device=dev)
        # One split-K workspace + counter array serves every other step GEMM
        # (they run one after another on one stream and leave the counters zero).
        ws_max, cnt_max = 0, 0
        for n, k in ((3 * D, D), (D, D), (4 * D, D), (D, 4 * D), (V, D)):
            wb, nc = ctypes.c_int64(), ctypes.c_int64()
            _lib.check(lib.cgpt_gemm_skinny_workspace(B, n, k, _DT[act], ctypes.byref(wb),
                                                      ctypes.byref(nc)), "skinny workspace")
            ws_max, cnt_max = max(ws_max, wb.value), max(cnt_max, nc.value)
        self.ws = torch.empty(max(ws_max // 4, 4), dtype=torch.float32, device=dev)
        self.ws_bytes = self.ws.numel() * 4
        self.counters = torch.zeros(max(cnt_max, 1), dtype=torch.int32, device=dev)

    @property
    def model(self):
        m = self._model()
        if m is None:
            raise RuntimeError("the model of this DecodeSession no longer exists")
        return m

    # ----------------------------------------------------------------- prefill

    def prefill(self, idx: torch.Tensor) -> None:
        """Run the prompt, fill the cache; leaves the last position's logits in
        ``self.logits``."""
        self.model._forward(idx, cache=self.cache, logits_out=self.logits)

    def greedy_first(self) -> None:
        """First new token (history column 0) from the prefill logits."""
        lib = _lib.load()
        s = torch.cuda.current_stream(self.model.device).cuda_stream
        V = self.model.config.vocab_size
        _lib.check(lib.cgpt_argmax(self.logits.data_ptr(), self.B, V, V, _DT[self.logits.dtype],
                                   self.ids.data_ptr(), self.hist.data_ptr(), self.max_new, None, s),
                   "argmax")

    # -------------------------------------------------------------------- step

    def step_logits(self) -> None:
        """One step for the tokens in ``self.ids`` at position t0 + step:
        appends to the cache and writes next-token logits to ``self.logits``."""
        m = self.model
        cfg = m.config
        lib = _lib.load()
        chk = _lib.check
        W = m.weights
        B, D, H, V, hd = self.B, cfg.n_embd, cfg.n_head, cfg.vocab_size, self.hd
        ac = _DT[m.dtype]
        f32 = _lib.CGPT_F32
        s = torch.cuda.current_stream(m.device).cuda_stream
        px, ph, pq, pa, pd, pf = (t.data_ptr() for t in (self.x, self.h, self.qkv, self.att,
                                                         self.delta, self.f))
        pstep = self.step.data_ptr()
        esz = self.qkv.element_size()

        pws, pcnt, nws, ncnt = (self.ws.data_ptr(), self.counters.data_ptr(), self.ws_bytes,
                                self.counters.numel())

        def gemm(a_ptr, w, b, c_ptr, n, k, epi, out_code, split=True):
            # split=False: the unsplit kernel, whose wider blocks suit the wide
            # GEMMs (c_fc, the LM head) better than the cross-block fix-up.
            chk(lib.cgpt_gemm_skinny(a_ptr, w.data_ptr(), None if b is None else b.data_ptr(),
                                     c_ptr, B, n, k, k, w.stride(0), n, ac, ac, out_code, epi,
                                     pws if split else None, nws, pcnt if split else None, ncnt,
                                     s), "gemm_skinny")

        def add_ln(delta_ptr, wk, keep_x=True):
            chk(lib.cgpt_add_layernorm(px, delta_ptr, px if delta_ptr and keep_x else None,
                                       W[wk + ".weight"].data_ptr(), W[wk + ".bias"].data_ptr(),
                                       ph, B, D, 1e-5, f32, f32, ac, ac, s), "add_layernorm")

        pp = self.parts.data_ptr()

        def gemm_parts(a_ptr, w, n, k):
            ns = self.splits[(n, k)]
            chk(lib.cgpt_gemm_partials(a_ptr, w.data_ptr(), pp, B, n, k, k, w.stride(0), n, ns,
                                       ac, s), "gemm_partials")
            return ns

        def add_ln_parts(ns, bias, wk, keep_x=True):
            chk(lib.cgpt_add_layernorm_partials(px, pp, ns, B * D, D, bias.data_ptr(),
                                                px if keep_x else None,
                                                W[wk + ".weight"].data_ptr(),
                                                W[wk + ".bias"].data_ptr(), ph, B, D, 1e-5, f32,
                                                f32, ac, ac, s), "add_layernorm_partials")

        chk(lib.cgpt_embedding_layernorm(self.ids.data_ptr(), W["wte"].data_ptr(),
                                         W["wpe"].data_ptr(), pstep, px,
                                         W["h.0.ln_1.weight"].data_ptr(),
                                         W["h.0.ln_1.bias"].data_ptr(), ph, B, 1, D, V, self.t0,
                                         cfg.block_size, 1e-5, ac, ac, self.err.data_ptr(), s),
            "embedding_layernorm")
        csb, csh, cst = self.cache.strides()
        t_max = self.cache.t_max
        scale = 1.0 / math.sqrt(hd)
        for i in range(cfg.n_layer):
            p = f"h.{i}."
            last = i + 1 == cfg.n_layer
            ln_next = "ln_f" if last else f"h.{i + 1}.ln_1"
            if self.partials:
                ns = gemm_parts(ph, W[p + "attn.c_attn.weight"], 3 * D, D)
                chk(lib.cgpt_attention_decode_partials(
                    pp, ns, B * 3 * D, 3 * D, W[p + "attn.c_attn.bias"].data_ptr(), 0, D, 2 * D,
                    self.cache.k[i].data_ptr(), self.cache.v[i].data_ptr(), pa, B, H, hd, t_max,
                    self.t0, pstep, csb, csh, cst, D, hd, scale, ac, self.err.data_ptr(), s),
                    "attention_decode_partials")
                ns = gemm_parts(pa, W[p + "attn.c_proj.weight"], D, D)
                add_ln_parts(ns, W[p + "attn.c_proj.bias"], p + "ln_2")
                # c_fc as split-K partials, then bias + GELU in one pass over them
                # (the GEMM's own fix-up would cost three dependent round trips).
                ns = gemm_parts(ph, W[p + "mlp.c_fc.weight"], 4 * D, D)
                chk(lib.cgpt_partials_bias_act(pp, ns, B * 4 * D, 4 * D,
                                               W[p + "mlp.c_fc.bias"].data_ptr(), ac, pf, 4 * D,
                                               B, 4 * D, _lib.EPI_BIAS_GELU, ac, s),
                    "partials_bias_act")
                ns = gemm_parts(pf, W[p + "mlp.c_proj.weight"], D, 4 * D)
                add_ln_parts(ns, W[p + "mlp.c_proj.bias"], ln_next, keep_x=not last)
                continue
            gemm(ph, W[p + "attn.c_attn.weight"], W[p + "attn.c_attn.bias"], pq, 3 * D, D,
                 _lib.EPI_BIAS, ac)
            chk(lib.cgpt_attention_decode(pq, pq + D * esz, pq + 2 * D * esz,
                                          self.cache.k[i].data_ptr(), self.cache.v[i].data_ptr(),
                                          pa, B, H, hd, t_max, self.t0, pstep,
                                          3 * D, hd, 3 * D, hd, 3 * D, hd, csb, csh, cst, D, hd,
                                          scale, ac, self.err.data_ptr(), s), "attention_decode")
            gemm(pa, W[p + "attn.c_proj.weight"], W[p + "attn.c_proj.bias"], pd, D, D,
                 _lib.EPI_BIAS, f32)
            add_ln(pd, p + "ln_2")
            gemm(ph, W[p + "mlp.c_fc.weight"], W[p + "mlp.c_fc.bias"], pf, 4 * D, D,
                 _lib.EPI_BIAS_GELU, ac)
            gemm(pf, W[p + "mlp.c_proj.weight"], W[p + "mlp.c_proj.bias"], pd, D, 4 * D,
                 _lib.EPI_BIAS, f32)
            add_ln(pd, ln_next, keep_x=not last)
        gemm(ph, W["lm_head.weight"], None, self.logits.data_ptr(), V, D, _lib.EPI_NONE,
             _DT[self.logits.dtype], split=not self.partials)

    def greedy_step(self) -> None:
        """``step_logits`` + argmax into ``ids`` and history column step + 1,
        then advance the step counter."""
        self.step_logits()
        lib = _lib.load()
        s = torch.cuda.current_stream(self.model.device).cuda_stream
        V = self.model.config.vocab_size
        _lib.check(lib.cgpt_argmax(self.logits.data_ptr(), self.B, V, V, _DT[self.logits.dtype],
                                   self.ids.data_ptr(), self.hist.data_ptr() + 8, self.max_new,
                                   self.step.data_ptr(), s), "argmax")
        self.step.add_(1)

    def _weights_key(self):
        m = self.model
        return (m.logits_dtype, tuple((k, t.data_ptr()) for k, t in m.weights.items()))

    def matches(self, B: int, t0: int, max_new: int) -> bool:
        """Whether this session can serve a generation of B sequences with a
        t0-token prompt and max_new new tokens: same shapes, and the model
        still holds the weight tensors (and logits dtype) any captured graph
        was recorded over."""
        return ((B, t0, max_new) == (self.B, self.t0, self.max_new) and
                self.logits.dtype == self.model.logits_dtype and
                (self._captured_over is None or self._captured_over == self._weights_key()))

    def _capture(self, fn) -> torch.cuda.CUDAGraph:
        """Capture ``fn`` outside inference mode: torch allocates its graph
        RNG state on the first capture while no graph is alive, and a graph
        kept by the session would otherwise leave that state an inference
        tensor that later captures outside inference mode cannot update."""
        dev = self.model.device
        # Dead objects that hold HIP graphs or memory are freed now, and no
        # collection runs during the capture (destroying a graph then fails).
        gc.collect()
        was_enabled = gc.isenabled()
        gc.disable()
        try:
            with torch.inference_mode(False):
                g = torch.cuda.CUDAGraph()
                side = torch.cuda.Stream(dev)
                side.wait_stream(torch.cuda.current_stream(dev))
                with torch.cuda.stream(side):
                    with torch.cuda.graph(g, stream=side):
                        fn()
                torch.cuda.current_stream(dev).wait_stream(side)
        finally:
            if was_enabled:
                gc.enable()
        self._captured_over = self._weights_key()
        return g

    def run_greedy(self, use_graph: bool = True) -> torch.Tensor:
        """Generate ``max_new`` tokens after ``prefill``; returns (B, max_new).
        The step graph captured by an earlier call on this session is
        replayed again (the step counter restarts at 0)."""
        self.step.zero_()
        self.err.zero_()
        self.greedy_first()
        n = self.max_new - 1
        if n <= 0:
            return self.hist
        if not use_graph or n < 3:
            for _ in range(n):
                self.greedy_step()
            return self.hist
        if self.graph is None:
            self.greedy_step()  # eager first step (also loads every kernel)
            self.graph = self._capture(self.greedy_step)
            n -= 1
        for _ in range(n):
            self.graph.replay()
        return self.hist

    def next_logits(self, use_graph: bool = True) -> None:
        """``step_logits`` for a caller that picks the tokens itself
        (sampling).  With ``use_graph`` the first call runs eagerly and
        captures the step; later calls on the session replay it."""
        if not use_graph:
            self.step_logits()
        elif self.graph_logits is not None:
            self.graph_logits.replay()
        else:
            self.step_logits()
            self.graph_logits = self._capture(self.step_logits)
