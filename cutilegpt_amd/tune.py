"""Tile sweep for the GEMM planner (``tiles.TABLE``).

Times every tile configuration of ``cgpt_gemm`` on the GEMM shapes of a
model's prefill forward and prints, per shape, the average launch time of
each tile and the winner, plus the ``TABLE`` entries the winners give.
Replaces the reference's fixed per-wrapper tile constants
(``cutile_gpt/kernels/linear.py:148-152,208-212``) and its unwired tile config
(``cutile_gpt/api/config.py:36-64``) with measured choices.

    python -m cutilegpt_amd.tune [--configs gpt2 medium xl] [--iters 10]

Each (shape, tile) is launched ``warmup`` times, then ``iters`` times back to
back from one captured HIP graph between two HIP events on the launch stream
(inputs hot in L2/MALL, the same way for every tile; the graph keeps host
launch overhead out of short kernels' times).  The residual-epilogue shapes (attn c_proj, MLP
c_proj: C += A W^T + bias into the fp32 residual stream) sweep the tiles that
epilogue runs on: the register-staged tiles 0-4, the slab kernel (14) and the
small pipeline tiles (17-19).
Needs a GPU.
"""

from __future__ import annotations

import argparse
import json
import sys
from typing import Dict, List, Tuple

from . import _lib

# name -> (n_embd, rows M of the prefill forward); vocabulary padded to 50304.
CONFIGS: Dict[str, Tuple[int, int]] = {
    "gpt2": (768, 16 * 1024),     # GPT-2 124M, b16 x s1024 (the benchmark)
    "medium": (512, 16 * 256),    # the reference's 'medium' preset, b16 x s256
    "xl": (1600, 32 * 128),       # GPT-2 XL prefill inside generate, b32 x 128
}
VOCAB_PAD = 50304
RESID_TILES = [0, 1, 2, 3, 4, 14, 17, 18, 19]


def shapes(name: str) -> List[Tuple[str, int, int, int, int, int]]:
    """(tag, M, N, K, epilogue, out dtype) of every GEMM in the forward."""
    d, m = CONFIGS[name]
    bf, f32 = _lib.CGPT_BF16, _lib.CGPT_F32
    return [
        ("c_attn", m, 3 * d, d, _lib.EPI_BIAS, bf),
        ("attn_c_proj", m, d, d, _lib.EPI_BIAS_RESID, f32),
        ("c_fc_gelu", m, 4 * d, d, _lib.EPI_BIAS_GELU, bf),
        ("mlp_c_proj", m, d, 4 * d, _lib.EPI_BIAS_RESID, f32),
        ("lm_head", m, VOCAB_PAD, d, _lib.EPI_NONE, f32),
    ]


def sweep(name: str, iters: int, warmup: int, out=sys.stdout):
    import torch

    lib = _lib.load()
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev)
    ntiles = lib.cgpt_gemm_num_tiles()
    g = torch.Generator(device=dev).manual_seed(0)
    winners = {}
    rows = []
    for tag, m, n, k, epi, oc in shapes(name):
        a = (torch.randn(m, k, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        w = (torch.randn(n, k, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        b = (torch.randn(n, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        c = torch.zeros(m, n, device=dev,
                        dtype=torch.float32 if oc == _lib.CGPT_F32 else torch.bfloat16)
        tiles = RESID_TILES if epi == _lib.EPI_BIAS_RESID else list(range(ntiles))
        fl = 2.0 * m * n * k
        best = None
        for t in tiles:
            def run():
                # On the current stream: the graph capture below records on its own.
                return lib.cgpt_gemm(a.data_ptr(), w.data_ptr(), b.data_ptr(), c.data_ptr(), m,
                                     n, k, k, k, n, _lib.CGPT_BF16, _lib.CGPT_BF16, oc, epi, t,
                                     torch.cuda.current_stream(dev).cuda_stream)
            if run() != 0:
                continue
            for _ in range(warmup):
                run()
            # The timed launches are replayed from a captured graph, so a short
            # kernel is not timed at the rate the host can launch it.
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(iters):
                    run()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(st)
            graph.replay()
            e1.record(st)
            torch.cuda.synchronize()
            del graph
            ms = e0.elapsed_time(e1) / iters
            rows.append((name, tag, m, n, k, t, ms, fl / ms / 1e9))
            print(f"{name:7s} {tag:12s} M={m:6d} N={n:6d} K={k:5d} tile {t:2d}: "
                  f"{ms * 1e3:9.1f} us {fl / ms / 1e9:7.1f} TFLOP/s", file=out, flush=True)
            if best is None or ms < best[1]:
                best = (t, ms)
        if epi == _lib.EPI_BIAS_RESID and c.dtype == torch.float32:
            c.zero_()  # keep the residual buffer finite after many in-place adds
        if best is not None:
            winners[(m, n, k)] = (tag, best[0], best[1], fl / best[1] / 1e9)
        del a, w, b, c
        torch.cuda.synchronize()
    return winners, rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--configs", nargs="+", default=sorted(CONFIGS), choices=sorted(CONFIGS))
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    args = ap.parse_args(argv)
    table = {}
    for name in args.configs:
        winners, _ = sweep(name, args.iters, args.warmup)
        for (m, n, k), (tag, t, ms, tf) in winners.items():
            print(f"winner {name:7s} {tag:12s} ({m}, {n}, {k}): tile {t} "
                  f"{ms * 1e3:.1f} us {tf:.1f} TFLOP/s", flush=True)
            table[f"{name}:{tag}"] = {"M": m, "N": n, "K": k, "tile": t,
                                      "us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1)}
    print(json.dumps(table), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
