"""Model parity on the GPU: CutileGPT.forward / generate against the CPU oracle
and the golden fixture, at the benchmark configurations.

Criteria (from the benchmark definition):
  fp32: max |logit error| <= 1e-3.
  bf16: max |logit error| <= 3e-2 against the exact (fp64) forward and against
        the oracle's bf16 flow.  Top-1 agreement is measured and reported;
        with random N(0, 0.02) weights the top-1/top-2 logit gap (~0.13) is
        within ~50x of the bf16 rounding noise (~2e-3), so the oracle's own
        bf16 flow run in fp32 vs fp64 arithmetic agrees on ~99.2% of positions.
        The bound asserted here, >= 98.5% of all positions and every
        last position, is what any bf16 implementation of this model can meet.
"""

import os

import numpy as np
import pytest
import torch

from cutilegpt_amd import CutileGPT, GPTConfig
from oracle import gpt_ref as R

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "nano_seed0.npz")


def make_model(cfg, w, dtype):
    m = CutileGPT(cfg, dtype=dtype, seed=0)
    m.load_weights(w)
    return m


def agreement(a, b):
    return (a.argmax(-1) == b.argmax(-1)).double().mean().item()


def test_nano_fp32_vs_golden_and_oracle(gpu):
    gold = np.load(GOLDEN)
    cfg = GPTConfig(n_layer=3, n_head=3, n_embd=48, block_size=1024)
    w = R.init_weights(3, 3, 48, seed=0)
    m = make_model(cfg, w, torch.float32)
    ids = torch.from_numpy(gold["ids"])
    logits, none = m(ids.to(gpu))
    assert none is None and logits.shape == (1, 64, 50257) and logits.dtype == torch.float32
    out = logits[0].double().cpu()
    assert np.abs(out[-1].numpy() - gold["last_logits"]).max() <= 1e-3
    assert np.array_equal(out.argmax(-1).numpy(), gold["argmax"])
    exact = R.gpt_forward(w, ids, 3, R.FLOWS["fp64"])[0]
    err = (out - exact).abs().max().item()
    print(f"nano fp32 max |err| = {err:.3e}")
    assert err <= 1e-3


def test_nano_greedy_generate_matches_golden(gpu):
    gold = np.load(GOLDEN)
    cfg = GPTConfig(n_layer=3, n_head=3, n_embd=48, block_size=1024)
    m = make_model(cfg, R.init_weights(3, 3, 48, seed=0), torch.float32)
    out = m.generate(torch.from_numpy(gold["greedy_prompt"]).to(gpu), 8, top_k=1)
    assert np.array_equal(out.cpu().numpy(), gold["greedy_out"])


def check_bf16(m, w, ids, n_head, label, rows=None):
    logits, _ = m(ids.to(ids.device if ids.is_cuda else "cuda"))
    out = logits.double().cpu()
    sel = slice(None) if rows is None else rows
    ids_cpu = ids.cpu()[sel]
    out = out[sel]
    exact = R.gpt_forward(w, ids_cpu, n_head, R.FLOWS["fp64"])
    flow = R.gpt_forward(w, ids_cpu, n_head, R.FLOWS["bf16"]).double()
    e_exact = (out - exact).abs().max().item()
    e_flow = (out - flow).abs().max().item()
    agree_all = agreement(out, exact)
    agree_last = agreement(out[:, -1], exact[:, -1])
    ref_agree = agreement(flow, exact)
    print(f"{label}: max|err| vs fp64 {e_exact:.3e}, vs bf16 flow {e_flow:.3e}; top-1 agree "
          f"{agree_all * 100:.3f}% (oracle bf16 flow itself {ref_agree * 100:.3f}%), last pos "
          f"{agree_last * 100:.1f}%")
    assert e_exact <= 3e-2 and e_flow <= 3e-2
    assert agree_all >= 0.985 and agree_last == 1.0


def test_medium_bf16(gpu):
    """'medium' GPT (8 layers, 8 heads, d 512), bf16 N(0,0.02) weights, b16 x s256."""
    cfg = GPTConfig(n_layer=8, n_head=8, n_embd=512, block_size=1024)
    w = R.init_weights(8, 8, 512, seed=0, dtype=torch.bfloat16)
    m = make_model(cfg, w, torch.bfloat16)
    ids = torch.randint(0, 50257, (16, 256), generator=torch.Generator().manual_seed(1))
    check_bf16(m, w, ids, 8, "medium b16xs256")


def test_gpt2_bf16_full_batch(gpu):
    """GPT-2 124M, bf16, b16 x s1024 on the GPU; sequences are independent, so the
    CPU oracle checks 2 of the 16 rows of the full-size batch."""
    cfg = GPTConfig.gpt2()
    w = R.init_weights(12, 12, 768, seed=0, dtype=torch.bfloat16)
    m = make_model(cfg, w, torch.bfloat16)
    ids = torch.randint(0, 50257, (16, 1024), generator=torch.Generator().manual_seed(2))
    check_bf16(m, w, ids, 12, "gpt2 b16xs1024 (rows 0 and 15)", rows=[0, 15])


def test_gpt2_hf_checkpoint_load(gpu, tmp_path):
    """Loader boundary: weights written as an HF GPT-2 directory, loaded through
    load_from_huggingface, give the same logits as loading the dict directly."""
    from cutilegpt_amd.hf_loader import save_hf_checkpoint
    cfg = GPTConfig(n_layer=2, n_head=4, n_embd=128, block_size=1024)
    w = R.init_weights(2, 4, 128, seed=5, dtype=torch.bfloat16)
    save_hf_checkpoint(str(tmp_path), w, cfg)
    a = CutileGPT(cfg, dtype=torch.bfloat16, seed=1)
    a.load_from_huggingface(str(tmp_path))
    b = make_model(cfg, w, torch.bfloat16)
    ids = torch.randint(0, 50257, (2, 33), generator=torch.Generator().manual_seed(3)).to(gpu)
    assert torch.equal(a(ids)[0], b(ids)[0])
    c = CutileGPT.from_pretrained(str(tmp_path), dtype=torch.bfloat16)
    assert torch.equal(c(ids)[0], b(ids)[0])


def test_ragged_lengths_fp32(gpu):
    """Sequence lengths that are not multiples of any tile, fp32 tolerance."""
    cfg = GPTConfig(n_layer=2, n_head=2, n_embd=64, block_size=1024)
    w = R.init_weights(2, 2, 64, seed=6)
    m = make_model(cfg, w, torch.float32)
    for T in (1, 2, 63, 65, 129, 200):
        ids = torch.randint(0, 50257, (3, T), generator=torch.Generator().manual_seed(T))
        out = m(ids.to(gpu))[0].double().cpu()
        err = (out - R.gpt_forward(w, ids, 2, R.FLOWS["fp64"])).abs().max().item()
        assert err <= 1e-3, (T, err)
