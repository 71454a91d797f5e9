"""Write the greedy-stream fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_streams.py [gpt2|xl|all]``).

The benchmark's bf16 criteria ask for greedy token streams identical to those of
"the reference's own implementation" for >= 95 % of sequences.  The reference
cannot run here (cuda.tile + CuPy + an NVIDIA GPU) and has no bf16 path at all
(CuPy has no bfloat16), so the expected streams come from the CPU oracle's
``bf16`` flow (``oracle.gpt_ref.FLOWS["bf16"]``): the same rounding points as the
HIP path (bf16 operands of every matrix product, fp32 residual stream and
projection outputs, GELU on the fp32 accumulator, fp32 logits), fp32
arithmetic.  The oracle's cached greedy loop (``generate_cached``) is pinned to
its full-recompute ``generate`` (the restatement of
``cutile_gpt/models/gpt.py:185-229``) in ``tests/test_oracle.py``.

Workloads (weights ``oracle.gpt_ref.init_weights(L, H, D, seed=0,
dtype=bfloat16)``: every Linear/embedding weight ~ N(0, 0.02), biases 0, LN
gamma 1 / beta 0; prompts ``randint(0, 50257, (B, 128))`` from
``torch.Generator().manual_seed(1)``; 128 greedy tokens):

* ``gpt2_bf16_streams.npz``  GPT-2 124M (12 layers, 12 heads, d 768), all
                             B = 32 prompts.
* ``xl_bf16_streams.npz``    GPT-2 XL (48 layers, 25 heads, d 1600), the
                             benchmark's B = 32 prompts; streams for the first
                             ``XL_ROWS`` of them (CPU time).

Each file holds ``prompts`` (B, 128) int64, ``streams`` (rows, 256) int64 (prompt
+ 128 tokens) and ``gap`` (rows, 128) float32: the oracle's top-1 minus top-2
logit at every step (a divergence at a step with a gap far below the bf16 noise
is a near-tie, not an error).
"""

import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import gpt_ref as R  # noqa: E402

PROMPT, NEW, BATCH = 128, 128, 32
XL_ROWS = 8
CONFIGS = {
    "gpt2": dict(L=12, H=12, D=768, rows=BATCH, file="gpt2_bf16_streams.npz"),
    "xl": dict(L=48, H=25, D=1600, rows=XL_ROWS, file="xl_bf16_streams.npz"),
}


def prompts(batch: int = BATCH) -> torch.Tensor:
    return torch.randint(0, 50257, (batch, PROMPT), generator=torch.Generator().manual_seed(1))


def weights(name: str) -> dict:
    c = CONFIGS[name]
    return R.init_weights(c["L"], c["H"], c["D"], seed=0, dtype=torch.bfloat16)


def make(name: str) -> None:
    c = CONFIGS[name]
    t0 = time.time()
    w = weights(name)
    # bf16 -> fp32 is exact; converting once keeps every step from re-widening
    # the whole model.
    w32 = {k: v.float() for k, v in w.items()}
    w32["lm_head.weight"] = w32["wte"]
    del w
    ids = prompts()[: c["rows"]]
    out, lg = R.generate_cached(w32, ids, c["H"], NEW, R.FLOWS["bf16"], return_logits=True)
    top2 = lg.float().topk(2, dim=-1).values
    gap = (top2[..., 0] - top2[..., 1]).numpy().astype(np.float32)
    path = os.path.join(HERE, c["file"])
    np.savez_compressed(path, prompts=prompts().numpy(), streams=out.numpy(), gap=gap)
    print(f"{name}: wrote {path} ({c['rows']} streams) in {time.time() - t0:.0f} s; "
          f"min gap {gap.min():.2e}")


if __name__ == "__main__":
    torch.set_num_threads(max(1, os.cpu_count() or 1))
    which = sys.argv[1] if len(sys.argv) > 1 else "all"
    for n in (CONFIGS if which == "all" else [which]):
        make(n)
