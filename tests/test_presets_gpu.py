"""Every ``GPTConfig`` preset's shape on the GPU against the fp64 oracle.

The presets (``cutile_gpt/models/config.py:19-87``) span head dims 16, 32 and
64, widths 48 to 1600 and block sizes 128 to 1024.  Each one here keeps its
head count, width and block size and is cut to two layers, with
checkpoint-like parameters (every bias ~N(0, 0.1), LayerNorm gamma ~N(1, 0.1),
beta ~N(0, 0.1), ``oracle.gpt_ref.randomize_affine``), and runs:

* the prefill forward at batch 2 and a ragged length (80 positions, not a
  multiple of the 64-key attention block; the nano preset's 128-position
  block size included), fp32 within 1e-3 of fp64 and bf16 within 3e-2 of the
  fp64 forward of the same bf16-valued weights (north_star's bars);
* for four presets, KV-cache greedy decoding in fp32, token for token equal
  to the oracle's full-recompute greedy stream.

Measured on MI355X (max |logit - fp64|): fp32 2.3e-7 (nano) to 1.1e-5
(gpt2-xl width); bf16 1.5e-3 (nano) to 1.9e-2 (gpt2-xl width).
"""

import pytest
import torch

from cutilegpt_amd import CutileGPT, GPTConfig
from oracle import gpt_ref as R

pytestmark = pytest.mark.gpu

PRESETS = ["nano", "micro", "mini", "gpt2", "gpt2-medium", "gpt2-large", "gpt2-xl",
           "tile-small", "tile-medium", "tile-large"]


def _preset_model(name, dtype, seed):
    full = GPTConfig.from_name(name)
    cfg = GPTConfig(n_layer=2, n_head=full.n_head, n_embd=full.n_embd,
                    block_size=full.block_size)
    w = R.randomize_affine(R.init_weights(2, full.n_head, full.n_embd,
                                          block_size=full.block_size, seed=seed),
                           seed=seed + 1000)
    if dtype == torch.bfloat16:
        w = {k: v.to(torch.bfloat16).float() for k, v in w.items()}
    m = CutileGPT(cfg, dtype=dtype, init_weights=False)
    m.load_weights(w)
    return m, w, cfg


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 3e-2)])
@pytest.mark.parametrize("name", PRESETS)
def test_preset_shape_forward_vs_fp64(gpu, name, dtype, tol):
    seed = 100 + PRESETS.index(name)
    m, w, cfg = _preset_model(name, dtype, seed)
    T = min(cfg.block_size, 80)
    ids = torch.randint(0, cfg.vocab_size, (2, T), generator=torch.Generator().manual_seed(seed))
    out = m(ids.to(gpu))[0].double().cpu()
    ref = R.gpt_forward({k: v.double() for k, v in w.items()}, ids, cfg.n_head, R.FLOWS["fp64"])
    assert out.shape == ref.shape == (2, T, cfg.vocab_size)
    err = (out - ref).abs().max().item()
    print(f"preset {name} {str(dtype)[6:]}: max |logit - fp64| = {err:.3e}")
    assert err <= tol, (name, err)


@pytest.mark.parametrize("name", ["nano", "gpt2-medium", "gpt2-large", "tile-large"])
def test_preset_shape_greedy_stream_fp32(gpu, name):
    seed = 200 + PRESETS.index(name)
    m, w, cfg = _preset_model(name, torch.float32, seed)
    idx = torch.randint(0, cfg.vocab_size, (2, 7), generator=torch.Generator().manual_seed(seed))
    out = m.generate(idx.to(gpu), 8, top_k=1)
    assert torch.equal(out.cpu(), R.generate(w, idx, cfg.n_head, 8)), name
