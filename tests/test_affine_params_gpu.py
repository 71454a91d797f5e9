"""Checkpoint-like parameters end to end on the GPU: every bias ~N(0, 0.1),
every LayerNorm gamma ~N(1, 0.1) and beta ~N(0, 0.1), each tensor drawn
separately (``oracle.gpt_ref.randomize_affine``), written as an HF GPT-2
directory and read back through ``load_from_huggingface``, or handed over as a
minGPT state dict through ``load_from_mingpt``, then run through the prefill
forward and the KV-cache decode step against the fp64 oracle.

A trained checkpoint has all of these tensors; with zero biases and unit
LayerNorms a bias or LayerNorm routed to the wrong place (the reference maps
each at cutile_gpt/models/gpt.py:266-296 and uses it at :120-177) would go
unnoticed.  ``test_nano_fp32_affine_through_both_loaders`` also shows that
the comparison sees such slips: the oracle fed the same weights with two
tensors exchanged differs from the GPU's logits by far more than the bar.

Bars: fp32 max |logit error| <= 1e-3; bf16 as ``tests/parity.check_bf16``
with top-1 floors set just under the measured agreement (these parameters
narrow the logit range, so near-ties are more frequent than with the plain
benchmark weights).  Measured on MI355X: nano fp32 2.6e-7; GPT-2 1.23e-2,
top-1 98.83 % against fp64 and 98.44 % against the bf16 flow (the reference's
own bf16 flow: 2.72e-2, 93.9 %); medium 8.9e-3, 98.83 % / 99.15 % (reference
flow 2.20e-2, 95.7 %), 15 of 16 last positions (the reference flow's too).
"""

import pytest
import torch

from cutilegpt_amd import CutileGPT, GPTConfig
from cutilegpt_amd.decode import DecodeSession
from cutilegpt_amd.hf_loader import save_hf_checkpoint
from oracle import gpt_ref as R
from tests.mingpt_stub import MinGPTStub
from tests.parity import check_bf16

pytestmark = pytest.mark.gpu


def affine_weights(L, H, D, seed, dtype=torch.float32):
    return R.randomize_affine(R.init_weights(L, H, D, seed=seed, dtype=dtype), seed=seed + 1000)


def swapped(w, a, b):
    """``w`` with tensors ``a`` and ``b`` exchanged (a planted loader slip)."""
    out = dict(w)
    out[a], out[b] = w[b], w[a]
    return out


def test_nano_fp32_affine_through_both_loaders(gpu, tmp_path):
    L, H, D = 3, 3, 48
    cfg = GPTConfig(n_layer=L, n_head=H, n_embd=D, block_size=1024)
    w = affine_weights(L, H, D, seed=0)
    save_hf_checkpoint(str(tmp_path), w, cfg)
    a = CutileGPT(cfg, dtype=torch.float32, init_weights=False)
    a.load_from_huggingface(str(tmp_path))
    b = CutileGPT(cfg, dtype=torch.float32, init_weights=False)
    b.load_from_mingpt(MinGPTStub(w, L))
    ids = torch.randint(0, 50257, (2, 64), generator=torch.Generator().manual_seed(1))
    la = a(ids.to(gpu))[0].double().cpu()
    lb = b(ids.to(gpu))[0].double().cpu()
    assert torch.equal(la, lb)
    exact = R.gpt_forward(w, ids, H, R.FLOWS["fp64"])
    err = (la - exact).abs().max().item()
    print(f"nano fp32, checkpoint-like biases/LN: max |err| vs fp64 {err:.3e}")
    assert err <= 1e-3
    for x, y in (("h.0.attn.c_proj.bias", "h.0.mlp.c_proj.bias"),
                 ("h.1.ln_1.weight", "h.1.ln_2.weight"), ("h.2.ln_1.bias", "h.2.ln_2.bias"),
                 ("h.0.ln_1.bias", "h.1.ln_1.bias"), ("ln_f.weight", "h.2.ln_2.weight")):
        # A GPU forward with the slip would sit d away from the correct oracle,
        # beyond the bar plus the error measured above: the check catches it.
        d = (la - R.gpt_forward(swapped(w, x, y), ids, H, R.FLOWS["fp64"])).abs().max().item()
        assert d > 1e-3 + err, (x, y, d)
    # k and v thirds of the fused QKV bias exchanged (q <-> k alone moves these
    # logits by only 4e-4: the key bias adds a per-query constant to every
    # score, which the softmax cancels, so that slip is below the fp32 bar)
    qkv = dict(w)
    for i in range(L):
        bq, bk, bv = w[f"h.{i}.attn.c_attn.bias"].split(D)
        qkv[f"h.{i}.attn.c_attn.bias"] = torch.cat([bq, bv, bk])
    assert (la - R.gpt_forward(qkv, ids, H, R.FLOWS["fp64"])).abs().max().item() > 1e-3 + err


def test_gpt2_bf16_affine_hf_checkpoint(gpu, tmp_path):
    """GPT-2 124M through the HF directory loader, b16 x s1024 on the GPU; the
    oracle checks rows 0 and 1."""
    cfg = GPTConfig.gpt2()
    w = affine_weights(12, 12, 768, seed=0, dtype=torch.bfloat16)
    save_hf_checkpoint(str(tmp_path), w, cfg)
    m = CutileGPT(cfg, dtype=torch.bfloat16, init_weights=False)
    m.load_from_huggingface(str(tmp_path))
    ids = torch.randint(0, 50257, (16, 1024), generator=torch.Generator().manual_seed(2))
    check_bf16(m(ids.to(gpu))[0], w, ids, 12, "gpt2 affine b16xs1024 (rows 0, 1)",
               rows=[0, 1], floor=0.98)


def test_medium_bf16_affine_mingpt(gpu):
    """'medium' (8 layers, 8 heads, d 512) through load_from_mingpt, b16 x s256,
    every row against the oracle."""
    cfg = GPTConfig(n_layer=8, n_head=8, n_embd=512, block_size=1024)
    w = affine_weights(8, 8, 512, seed=0, dtype=torch.bfloat16)
    m = CutileGPT(cfg, dtype=torch.bfloat16, init_weights=False)
    m.load_from_mingpt(MinGPTStub(w, 8))
    assert m.weights["lm_head.weight"].data_ptr() == m.weights["wte"].data_ptr()
    ids = torch.randint(0, 50257, (16, 256), generator=torch.Generator().manual_seed(1))
    check_bf16(m(ids.to(gpu))[0], w, ids, 8, "medium affine b16xs256", floor=0.985,
               last=15 / 16)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 3e-2)])
def test_decode_steps_affine_vs_oracle(gpu, dtype, tol):
    """KV-cache decode (prefill, then greedy steps through the split-K GEMM
    partials, the decode attention with the QKV bias, and the residual +
    LayerNorm kernels that add the projection biases): every step's logits
    against the fp64 oracle on the tokens chosen."""
    L, H, D = 3, 4, 128
    cfg = GPTConfig(n_layer=L, n_head=H, n_embd=D, block_size=1024)
    w = affine_weights(L, H, D, seed=7, dtype=dtype)
    m = CutileGPT(cfg, dtype=dtype, init_weights=False)
    m.load_weights(w)
    B, T0, n = 3, 11, 9
    idx = torch.randint(0, 50257, (B, T0), generator=torch.Generator().manual_seed(8)).to(gpu)
    sess = DecodeSession(m, B, T0, n)
    sess.prefill(idx)
    seen = [sess.logits.double().cpu()]
    sess.greedy_first()
    for _ in range(n - 1):
        sess.greedy_step()
        seen.append(sess.logits.double().cpu())
    torch.cuda.synchronize()
    assert sess.err.item() == 0
    seq = torch.cat([idx, sess.hist], dim=1).cpu()
    exact = R.gpt_forward(w, seq[:, :-1], H, R.FLOWS["fp64"])
    for s, lg in enumerate(seen):
        e = (lg - exact[:, T0 - 1 + s]).abs().max().item()
        assert e <= tol, (s, e)
        assert torch.equal(sess.hist[:, s].cpu(), lg.argmax(-1))
