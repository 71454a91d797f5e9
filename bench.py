"""Prefill throughput of the GPT-2 forward hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload gpt2|medium|xl-decode|kernels]

Workload (default): GPT-2 124M architecture (12 layers, 12 heads, d 768, MLP 3072,
vocab 50257), bf16 random-init weights N(0, 0.02) written as an HF GPT-2
checkpoint directory and loaded through ``CutileGPT.load_from_huggingface``;
uniform random token ids; one step = one prefill forward of batch 16 x seq 1024
(16384 tokens) producing fp32 logits.  Inputs are resident on the GPU before
the timed region.  Prints one JSON line.

``roofline`` is the LM-head GEMM launch (the single largest launch: 2*16384*768*
50257 FLOP), timed with stream events around that launch inside the timed
steps.  ``cpu_baseline`` is the CPU oracle's fp32 forward of the same model
(a minGPT-architecture PyTorch forward) on the host cores, over a bounded
sample.  ``breakdown`` comes from one extra, separately timed forward with
events around every launch.

``standalone_kernels`` (also ``--workload kernels`` on its own): the standalone
kernel set — tanh-GELU, LayerNorm and causal attention in fp32 and bf16 — each
timed over rotating buffers larger than the MALL, as a fraction of its
roofline; the HBM-bound ones also beside plain device copies of the same bytes
timed the same way (``copy_variants_GB/s``: one-shot and persistent grids, 1-8
vectors in flight a thread, non-temporal and cached, and torch's copy_;
``copy_GB/s`` is the fastest, ``frac_of_copy`` the kernel against it): the rate
any copy reaches at 50-100 MB, below the 8 TB/s peak.

``--workload xl-decode``: KV-cache greedy decoding of GPT-2 XL (48 layers, 25
heads, d 1600), bf16 N(0, 0.02) weights generated on the device, batch 32,
prompt 128, 128 new tokens.  A step = one captured decode step (all 32
sequences advance one token), replayed from a HIP graph; ``value`` is steady
decode tok/s (32 / step time), ``e2e`` the whole ``generate`` call (prefill +
128 tokens).  ``roofline`` is HBM: the step's algorithmic bytes (every weight
once + the KV cache rows read) over the step time, and the LM-head skinny GEMM
alone.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
# Bytes beyond L2 per LM-head launch (2.0 x FETCH_SIZE + 1.0 x WRITE_SIZE, factors from
# a 1 GiB copy), measured with rocprofv3 --pmc on the GPT-2 workload; see
# profiles/lm_head_gemm_gpt2_traffic_pmc.md.  Only valid for the gpt2 workload.
LM_HEAD_TRAFFIC_BYTES = 5.15e9

# Kernel behind a persistent tile id (the LM head's roofline names it).
TILE_KERNELS = {
    14: "gemm_slab_kernel 256x192, fragment read-ahead, block-staged whole-line stores",
    16: "gemm_pipe_kernel 256x256, wave-staged whole-line non-temporal stores",
}

WORKLOADS = {
    "gpt2": dict(n_layer=12, n_head=12, n_embd=768, batch=16, seq=1024,
                 name="gpt2-124m prefill b16xs1024"),
    "medium": dict(n_layer=8, n_head=8, n_embd=512, batch=16, seq=256,
                   name="medium-8L-512 prefill b16xs256"),
}


def flops(L, D, B, T, V=50257):
    M = B * T
    gemm = L * 2 * M * D * (3 * D + D + 4 * D + 4 * D)
    head = 2 * M * D * V
    attn = L * 4 * B * D * T * (T + 1) // 2  # causal half incl. diagonal, all heads
    return gemm, head, attn


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="gpt2", choices=sorted(WORKLOADS) + ["xl-decode", "kernels"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seqs", type=int, default=8,
                    help="sequences (of seq_len tokens) per timed CPU-baseline forward")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB 3 times (a kernel of "
                         "known traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (every box has a single MI355X); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.workload == "xl-decode":
        bench_xl_decode(args)
        return
    if args.workload == "kernels":
        bench_kernels(args)
        return

    import torch
    from cutilegpt_amd import CutileGPT, GPTConfig, _lib
    from cutilegpt_amd.hf_loader import save_hf_checkpoint

    wl = WORKLOADS[args.workload]
    L, H, D, B, T = wl["n_layer"], wl["n_head"], wl["n_embd"], wl["batch"], wl["seq"]
    V = 50257
    cfg = GPTConfig(vocab_size=V, block_size=1024, n_layer=L, n_head=H, n_embd=D)
    dev = torch.device("cuda:0")

    # bf16 N(0, 0.02) weights (biases 0, LN 1/0) through the HF checkpoint loader.
    g = torch.Generator().manual_seed(0)
    w = {}
    bf = torch.bfloat16
    rn = lambda *s: (torch.randn(*s, generator=g) * 0.02).to(bf)
    w["wte"], w["wpe"] = rn(V, D), rn(1024, D)
    for i in range(L):
        p = f"h.{i}."
        w[p + "ln_1.weight"], w[p + "ln_1.bias"] = torch.ones(D, dtype=bf), torch.zeros(D, dtype=bf)
        w[p + "attn.c_attn.weight"], w[p + "attn.c_attn.bias"] = rn(3 * D, D), torch.zeros(3 * D, dtype=bf)
        w[p + "attn.c_proj.weight"], w[p + "attn.c_proj.bias"] = rn(D, D), torch.zeros(D, dtype=bf)
        w[p + "ln_2.weight"], w[p + "ln_2.bias"] = torch.ones(D, dtype=bf), torch.zeros(D, dtype=bf)
        w[p + "mlp.c_fc.weight"], w[p + "mlp.c_fc.bias"] = rn(4 * D, D), torch.zeros(4 * D, dtype=bf)
        w[p + "mlp.c_proj.weight"], w[p + "mlp.c_proj.bias"] = rn(D, 4 * D), torch.zeros(D, dtype=bf)
    w["ln_f.weight"], w["ln_f.bias"] = torch.ones(D, dtype=bf), torch.zeros(D, dtype=bf)
    w["lm_head.weight"] = w["wte"]
    model = CutileGPT(cfg, dtype=bf, seed=0)
    with tempfile.TemporaryDirectory() as ckpt:
        save_hf_checkpoint(ckpt, w, cfg)
        model.load_from_huggingface(ckpt)
    ids = torch.randint(0, V, (B, T), generator=torch.Generator().manual_seed(1)).to(dev)
    print(f"[bench] workload {wl['name']}: warmup {args.warmup}, steps {args.steps}",
          file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        model(ids)
    torch.cuda.synchronize()

    # Timed region: K forwards; events around the LM-head launch only.
    stream = torch.cuda.current_stream()
    head_ev = []

    def head_probe(tag, start):
        if tag == "lm_head":
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(stream)
            head_ev.append(ev)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.forward(ids, probe=head_probe)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    head_ms = [head_ev[2 * i].elapsed_time(head_ev[2 * i + 1]) for i in range(args.steps)]
    head_avg_ms = sum(head_ms) / len(head_ms)
    ms_per_step = elapsed * 1e3 / args.steps
    tokens = B * T
    tok_s = tokens * args.steps / elapsed
    gemm_f, head_f, attn_f = flops(L, D, B, T, V)
    head_tflops = head_f / (head_avg_ms * 1e-3) / 1e12

    # Breakdown: one more forward, events around every launch.
    marks = []

    def all_probe(tag, start):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(stream)
        marks.append((tag, start, ev))

    model.forward(ids, probe=all_probe)
    torch.cuda.synchronize()
    per = {}
    for i in range(0, len(marks), 2):
        tag, _, e0 = marks[i]
        per.setdefault(tag, [0.0, 0])
        per[tag][0] += e0.elapsed_time(marks[i + 1][2])
        per[tag][1] += 1
    M = B * T
    work = {  # algorithmic FLOP (GEMM/attention) or bytes (LN/embedding) per forward
        "gemm_qkv": ("TFLOP/s", L * 2 * M * D * 3 * D),
        "gemm_proj": ("TFLOP/s", L * 2 * M * D * D),
        "gemm_fc_gelu": ("TFLOP/s", L * 2 * M * D * 4 * D),
        "gemm_mlp_proj": ("TFLOP/s", L * 2 * M * 4 * D * D),
        "lm_head": ("TFLOP/s", head_f),
        "attention": ("TFLOP/s", attn_f),
        # LN: read x fp32, write y bf16 (the residual adds live in the projection
        # GEMMs' epilogues)
        "ln": ("GB/s", 2 * L * M * D * (4 + 2)),
        # gather + layer 0's LN: read wte + wpe rows bf16, write x fp32 + y bf16
        "embedding": ("GB/s", M * D * (2 + 2 + 4 + 2)),
    }
    breakdown = {}
    for tag, (ms, n) in per.items():
        unit, amount = work[tag]
        rate = amount / (ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
        peak = PEAK_BF16_TFLOPS if unit == "TFLOP/s" else PEAK_HBM_GBS
        breakdown[tag] = {"ms": round(ms, 4), "launches": n, unit: round(rate, 1),
                          "frac": round(rate / peak, 4)}

    if args.calib_copy_mib > 0:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # The standalone kernel set (GELU / LayerNorm / attention, fp32 and bf16).
    standalone = standalone_kernels() if args.workload == "gpt2" else None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w, ids, H, args.cpu_seqs)

    from cutilegpt_amd.tiles import gemm_tile
    Vp = model._head_pad.shape[0]
    head_tile = gemm_tile(_lib.CGPT_BF16, B * T, Vp, D)
    head_kernel = (f"lm_head GEMM (tile {head_tile}: {TILE_KERNELS.get(head_tile, 'library choice')}; "
                   f"bf16 in, fp32 out, M={B * T}, N={V} padded to {Vp}, K={D})")
    metric = ("prefill tok/s (GPT-2 124M, b16×s1024, bf16) + % of MFMA/HBM roofline"
              if args.workload == "gpt2" else f"prefill tok/s ({wl['name']}, bf16)")
    line = {
        "metric": metric,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random N(0,0.02) bf16 weights via HF-format checkpoint, uniform ids)",
        "config": {"workload": wl["name"], "n_layer": L, "n_head": H, "n_embd": D,
                   "vocab_size": V, "batch": B, "seq_len": T, "logits": "fp32",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": head_kernel,
                     "achieved": round(head_tflops, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(head_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": LM_HEAD_TRAFFIC_BYTES if args.workload == "gpt2" else None,
                     "avg_launch_ms": round(head_avg_ms, 4)},
        "forward_tflops": round((gemm_f + head_f + attn_f) / (ms_per_step * 1e-3) / 1e12, 1),
        "breakdown": breakdown,
        "standalone_kernels": standalone,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_xl_decode(args):
    """GPT-2 XL KV-cache greedy decode, b32, prompt 128 + 128 new tokens."""
    import statistics

    import torch
    from cutilegpt_amd import CutileGPT, GPTConfig, _lib
    from cutilegpt_amd.decode import DecodeSession

    L, H, D, B, T0, NEW, V = 48, 25, 1600, 32, 128, 128, 50257
    hd = D // H
    cfg = GPTConfig(vocab_size=V, block_size=1024, n_layer=L, n_head=H, n_embd=D)
    dev = torch.device("cuda:0")
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(0)
    rn = lambda *s: (torch.randn(*s, generator=g, device=dev) * 0.02).to(bf)
    ones = lambda n: torch.ones(n, dtype=bf, device=dev)
    zeros = lambda n: torch.zeros(n, dtype=bf, device=dev)
    w = {"wte": rn(V, D), "wpe": rn(1024, D), "ln_f.weight": ones(D), "ln_f.bias": zeros(D)}
    for i in range(L):
        p = f"h.{i}."
        w[p + "ln_1.weight"], w[p + "ln_1.bias"] = ones(D), zeros(D)
        w[p + "attn.c_attn.weight"], w[p + "attn.c_attn.bias"] = rn(3 * D, D), zeros(3 * D)
        w[p + "attn.c_proj.weight"], w[p + "attn.c_proj.bias"] = rn(D, D), zeros(D)
        w[p + "ln_2.weight"], w[p + "ln_2.bias"] = ones(D), zeros(D)
        w[p + "mlp.c_fc.weight"], w[p + "mlp.c_fc.bias"] = rn(4 * D, D), zeros(4 * D)
        w[p + "mlp.c_proj.weight"], w[p + "mlp.c_proj.bias"] = rn(D, 4 * D), zeros(D)
    model = CutileGPT(cfg, dtype=bf, init_weights=False)
    model.load_weights(w)
    del w
    ids = torch.randint(0, V, (B, T0), generator=torch.Generator().manual_seed(1)).to(dev)
    print(f"[bench] workload gpt2-xl decode b{B} {T0}+{NEW}: warmup {args.warmup}, "
          f"steps {args.steps}", file=sys.stderr, flush=True)

    # End to end: generate() = prefill + 128 greedy tokens (graph replay).
    for _ in range(max(1, args.warmup // 5)):
        model.generate(ids, NEW, top_k=1)
    torch.cuda.synchronize()
    e2e = []
    for _ in range(3):
        t0 = time.perf_counter()
        out = model.generate(ids, NEW, top_k=1)
        torch.cuda.synchronize()
        e2e.append(time.perf_counter() - t0)
    e2e_s = statistics.median(e2e)

    # Steady decode: one captured step replayed; the step counter is reset so
    # every replay sees the same positions (T0 .. T0+K-1 cycle).
    sess = DecodeSession(model, B, T0, NEW)
    sess.prefill(ids)
    sess.greedy_first()
    sess.greedy_step()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.graph(graph, stream=side):
        sess.greedy_step()
    torch.cuda.current_stream(dev).wait_stream(side)
    k = min(args.steps, NEW - 2)
    for _ in range(args.warmup):
        sess.step.fill_(1)
        graph.replay()
    sess.step.fill_(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(k):
        graph.replay()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / k
    mean_ctx = T0 + 1 + (k - 1) / 2.0 + 1  # keys visible per step, averaged

    # LM-head skinny GEMM alone (the single largest launch of a step), called as
    # the step calls it (no split-K workspace), alternating between the head and
    # a copy of it so that no launch finds its 161 MB of weights in the 256 MB
    # MALL (as in the step, where 3 GB of other weights pass in between).
    lib = _lib.load()
    st = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    head_ws = [model.weights["lm_head.weight"]]
    head_ws.append(head_ws[0].clone())
    use_ws = not sess.partials
    call = lambda i: _lib.check(lib.cgpt_gemm_skinny(
        sess.h.data_ptr(), head_ws[i % 2].data_ptr(), None, sess.logits.data_ptr(), B, V, D, D,
        head_ws[i % 2].stride(0), V, _lib.CGPT_BF16, _lib.CGPT_BF16, _lib.CGPT_F32,
        _lib.EPI_NONE, sess.ws.data_ptr() if use_ws else None, sess.ws_bytes,
        sess.counters.data_ptr() if use_ws else None, sess.counters.numel(), st.cuda_stream),
        "head")
    for i in range(4):
        call(i)
    ev0.record(st)
    for i in range(20):
        call(i)
    ev1.record(st)
    torch.cuda.synchronize()
    head_ms = ev0.elapsed_time(ev1) / 20
    head_bytes = V * D * 2 + B * D * 2 + B * V * 4

    weight_bytes = L * 12 * D * D * 2 + L * (3 * D + D + 4 * D + D + 4 * D) * 2 + V * D * 2
    kv_bytes = L * 2 * B * H * mean_ctx * hd * 2
    step_bytes = weight_bytes + kv_bytes
    line = {
        "metric": "decode tok/s (GPT-2 XL, b32, 128+128 greedy, bf16)",
        "value": round(B / step_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": k,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random N(0,0.02) bf16 weights generated on device, uniform ids)",
        "config": {"workload": "gpt2-xl decode b32 128+128 greedy", "n_layer": L, "n_head": H,
                   "n_embd": D, "vocab_size": V, "batch": B, "prompt": T0, "new_tokens": NEW,
                   "parallelism": "single GPU"},
        "e2e": {"generate_s": round(e2e_s, 4), "tok_s": round(B * NEW / e2e_s, 1),
                "what": "generate(top_k=1): prefill 32x128 + 128 tokens, graph replay"},
        "roofline": {"bound": "hbm", "kernel": "decode step (skinny GEMMs + decode attention)",
                     "achieved": round(step_bytes / step_s / 1e9, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(step_bytes / step_s / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": None, "bytes_per_step": int(step_bytes),
                     "lm_head_skinny": {"avg_launch_ms": round(head_ms, 4),
                                        "achieved_GBs": round(head_bytes / head_ms / 1e6, 1),
                                        "frac": round(head_bytes / head_ms / 1e6 / PEAK_HBM_GBS, 4)}},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


PEAK_FP32_TFLOPS = 157.3    # MI355X dense fp32 MFMA
# Rotating working set of the HBM-bound standalone kernels: several times the
# 256 MB MALL, so every launch streams from and to HBM.
ROTATE_BYTES = 640 << 20


def standalone_kernels(iters=40):
    """The standalone kernel set (tanh-GELU on 32x512x768, LayerNorm over 16384
    rows of 768 with gamma~N(1,0.1), beta~N(0,0.1), causal attention 12 heads x
    64 at batch 8 x seq 512), fp32 and bf16, inputs N(0,1) from seed 0.  Each
    kernel is launched ``iters`` times through the C ABI between two HIP events
    on the launch stream; GELU and LayerNorm rotate over copies of their
    buffers totalling ~ROTATE_BYTES so no launch reads what an earlier one left
    in the MALL.  Returns {name: {...}} with the average launch time and the
    achieved fraction of the kernel's roofline (HBM for GELU/LN, MFMA for
    attention)."""
    import torch
    from cutilegpt_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev)
    s = st.cuda_stream
    code = {torch.float32: _lib.CGPT_F32, torch.bfloat16: _lib.CGPT_BF16}

    def timed(launch, nbuf):
        for i in range(nbuf):
            launch(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for i in range(iters):
            launch(i % nbuf)
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    blib = ctypes.CDLL(os.path.join(os.path.dirname(_lib.LIB_PATH), "libcgpt_bench.so"))
    blib.cgpt_bench_copy_variant.restype = ctypes.c_int
    blib.cgpt_bench_copy_variant.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_void_p]
    # Plain copies of the same bytes (csrc_bench/ceiling.hip): (variant, 16-byte
    # vectors a thread, blocks a CU).  0 = one-shot grid, one vector a thread;
    # 1 = persistent grid, non-temporal; 2 = persistent, cached; 3 = one-shot,
    # consecutive vectors a thread.  The fastest of a sweep of 29 such copies at
    # 50 and 100 MB on MI355X are here, beside torch's own copy_.
    copy_variants = {"oneshot_v1": (0, 1, 1), "persistent_nt_v4_b8": (1, 4, 8),
                     "persistent_nt_v8_b4": (1, 8, 4), "persistent_nt_v8_b8": (1, 8, 8),
                     "persistent_cached_v4_b8": (2, 4, 8), "oneshot_consecutive_v2": (3, 2, 1)}

    def copy_ceiling(xs, ys, nbytes):
        # The rate plain device copies reach at the same byte count (read
        # nbytes / 2, write nbytes / 2), timed the same way over the same
        # rotating buffers; returns (best GB/s, {variant: GB/s}).
        rates = {}
        for name, (var, vec, bpc) in copy_variants.items():
            def one(i, var=var, vec=vec, bpc=bpc):
                if blib.cgpt_bench_copy_variant(xs[i].data_ptr(), ys[i].data_ptr(), nbytes // 2,
                                                var, vec, bpc, s) != 0:
                    raise RuntimeError("cgpt_bench_copy_variant failed")
            rates[name] = round(nbytes / timed(one, len(xs)) / 1e6, 1)
        rates["torch_copy_"] = round(nbytes / timed(lambda i: ys[i].copy_(xs[i]), len(xs)) / 1e6, 1)
        return max(rates.values()), rates

    def copies(t, pair_bytes):
        n = max(2, -(-ROTATE_BYTES // pair_bytes))
        return [t.clone() for _ in range(n)]

    g = torch.Generator().manual_seed(0)
    gelu_x = torch.randn(32, 512, 768, generator=g)
    ln_x = torch.randn(16384, 768, generator=g)
    ln_w = 1.0 + 0.1 * torch.randn(768, generator=g)
    ln_b = 0.1 * torch.randn(768, generator=g)
    qkv = [torch.randn(8, 12, 512, 64, generator=g) for _ in range(3)]
    out = {}
    for dt, tag in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        es = torch.finfo(dt).bits // 8
        # GELU: read n + write n elements.
        n = gelu_x.numel()
        xs = copies(gelu_x.to(dev, dt), 2 * n * es)
        ys = [torch.empty_like(xs[0]) for _ in xs]
        ms = timed(lambda i: _lib.check(lib.cgpt_gelu(xs[i].data_ptr(), ys[i].data_ptr(), n,
                                                      code[dt], s), "gelu"), len(xs))
        nbytes = 2 * n * es
        copy, rates = copy_ceiling(xs, ys, nbytes)
        out[f"gelu_{tag}"] = {"shape": [32, 512, 768], "avg_launch_ms": round(ms, 4),
                              "bytes": nbytes, "GB/s": round(nbytes / ms / 1e6, 1),
                              "frac": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4), "bound": "hbm",
                              "copy_GB/s": copy, "copy_frac_of_peak": round(copy / PEAK_HBM_GBS, 4),
                              "frac_of_copy": round(nbytes / ms / 1e6 / copy, 4),
                              "copy_variants_GB/s": rates}
        del xs, ys
        # LayerNorm: read x, write y, read gamma and beta.
        M, N = ln_x.shape
        xs = copies(ln_x.to(dev, dt), 2 * M * N * es)
        ys = [torch.empty_like(xs[0]) for _ in xs]
        gw, gb = ln_w.to(dev, dt), ln_b.to(dev, dt)
        ms = timed(lambda i: _lib.check(lib.cgpt_add_layernorm(
            xs[i].data_ptr(), None, None, gw.data_ptr(), gb.data_ptr(), ys[i].data_ptr(), M, N,
            1e-5, code[dt], 0, code[dt], code[dt], s), "layernorm"), len(xs))
        nbytes = 2 * M * N * es + 2 * N * es
        copy, rates = copy_ceiling(xs, ys, 2 * M * N * es)
        out[f"layernorm_{tag}"] = {"shape": [M, N], "avg_launch_ms": round(ms, 4),
                                   "bytes": nbytes, "GB/s": round(nbytes / ms / 1e6, 1),
                                   "frac": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
                                   "bound": "hbm", "copy_GB/s": copy,
                                   "copy_frac_of_peak": round(copy / PEAK_HBM_GBS, 4),
                                   "frac_of_copy": round(nbytes / ms / 1e6 / copy, 4),
                                   "copy_variants_GB/s": rates}
        del xs, ys
        # Causal attention, (B, H, T, hd) contiguous: 4*B*H*hd*T(T+1)/2 FLOP.
        B, H, T, hd = qkv[0].shape
        q, k, v = (t.to(dev, dt) for t in qkv)
        o = torch.empty_like(q)
        qs = q.stride()[:3]
        ms = timed(lambda i: _lib.check(lib.cgpt_attention_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, T, T, hd, *qs, *qs,
            *qs, *qs, 1.0 / math.sqrt(hd), 1, code[dt], s), "attention"), 1)
        fl = 4 * B * H * hd * T * (T + 1) // 2
        peak = PEAK_FP32_TFLOPS if dt == torch.float32 else PEAK_BF16_TFLOPS
        out[f"attention_{tag}"] = {"shape": [B, H, T, hd], "avg_launch_ms": round(ms, 4),
                                   "flop": fl, "TFLOP/s": round(fl / ms / 1e9, 1),
                                   "frac": round(fl / ms / 1e9 / peak, 4), "bound": "mfma",
                                   "peak_TFLOP/s": peak}
        del q, k, v, o
    torch.cuda.synchronize()
    return out


def bench_kernels(args):
    """``--workload kernels``: the standalone kernel set alone, one JSON line."""
    res = standalone_kernels(iters=max(args.steps, 10))
    fracs = [r["frac"] for r in res.values()]
    line = {
        "metric": "standalone kernel set (tanh-GELU 32x512x768, LayerNorm 16384x768, causal "
                  "attention b8 h12 s512 d64; fp32 and bf16): fraction of roofline",
        "value": round(sum(fracs) / len(fracs), 4),
        "unit": "mean frac of roofline over the 6 kernels",
        "n_gpus": 1, "steps": max(args.steps, 10), "warmup": 1,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32+bf16", "data": "synthetic N(0,1) inputs from seed 0",
        "config": {"workload": "standalone kernels", "rotate_bytes": ROTATE_BYTES},
        "kernels": res,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def cpu_model() -> str:
    """The host CPU's model name as lscpu reports it (``/proc/cpuinfo`` when
    lscpu is absent)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w, ids, n_head, n_seqs):
    """CPU oracle fp32 forward (minGPT-architecture PyTorch) on the host cores:
    1 warmup + 3 timed forwards of ``n_seqs`` sequences, median."""
    import torch
    from oracle import gpt_ref as R

    threads = torch.get_num_threads()
    w32 = {k: v.float() for k, v in w.items()}
    w32["lm_head.weight"] = w32["wte"]
    x = ids[:n_seqs].cpu()
    times = []
    with torch.inference_mode():
        R.gpt_forward(w32, x, n_head, R.FLOWS["fp32"])
        for _ in range(3):
            t0 = time.perf_counter()
            R.gpt_forward(w32, x, n_head, R.FLOWS["fp32"])
            times.append(time.perf_counter() - t0)
    med = sorted(times)[1]
    return {"value": round(x.numel() / med, 1), "unit": "tok/s", "cores": threads,
            "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{n_seqs} x {x.shape[1]} tokens per forward, fp32, 1 warmup + 3 timed, median "
                      f"{med:.2f} s (oracle.gpt_ref.gpt_forward, torch threads={threads}, "
                      f"os.cpu_count()={os.cpu_count()})"}


if __name__ == "__main__":
    main()
