"""Loader boundary on the GPU: load_from_mingpt (untied LM head),
HFWeightLoader.load on a local directory, a pytorch_model.bin checkpoint, and
the bf16-logits option of the forward.

References: cutile_gpt/models/gpt.py:306-343 (load_from_mingpt),
cutile_gpt/utils/hf_loader.py:42-67 (HFWeightLoader.load),
cutile_gpt/models/gpt.py:231-304 (load_from_huggingface)."""

import json
import os

import pytest
import torch

from cutilegpt_amd import CutileGPT, GPTConfig, HFWeightLoader
from cutilegpt_amd.hf_loader import internal_to_hf, save_hf_checkpoint
from oracle import gpt_ref as R
from tests.mingpt_stub import MinGPTStub

pytestmark = pytest.mark.gpu


def untied_weights(n_layer, n_head, n_embd, seed, dtype=torch.float32):
    w = R.init_weights(n_layer, n_head, n_embd, seed=seed, dtype=dtype)
    g = torch.Generator().manual_seed(seed + 100)
    w["lm_head.weight"] = (torch.randn(w["wte"].shape, generator=g) * 0.02).to(dtype)
    return w


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 3e-2)])
def test_load_from_mingpt_untied_head(gpu, dtype, tol):
    """The untied lm_head of a minGPT model is used as is (gpt.py:340); the
    logits match the oracle run with that separate head, and differ from a
    forward with the head tied to wte."""
    L, H, D = 2, 4, 128
    w = untied_weights(L, H, D, seed=21, dtype=dtype)
    cfg = GPTConfig(n_layer=L, n_head=H, n_embd=D, block_size=1024)
    m = CutileGPT(cfg, dtype=dtype, seed=0)
    m.load_from_mingpt(MinGPTStub(w, L))
    assert m.weights["lm_head.weight"] is not m.weights["wte"]
    ids = torch.randint(0, 50257, (2, 37), generator=torch.Generator().manual_seed(22))
    out = m(ids.to(gpu))[0].double().cpu()
    exact = R.gpt_forward(w, ids, H, R.FLOWS["fp64"])
    err = (out - exact).abs().max().item()
    print(f"load_from_mingpt {dtype}: max |err| vs untied-head oracle {err:.3e}")
    assert err <= tol
    tied = dict(w)
    tied["lm_head.weight"] = w["wte"]
    assert (out - R.gpt_forward(tied, ids, H, R.FLOWS["fp64"])).abs().max().item() > 10 * tol


def test_hf_weight_loader_local_directory(gpu, tmp_path):
    """HFWeightLoader(dir).load() returns the HF-keyed state dict on the device
    (Conv1D weights (in, out), as transformers stores them) and the sizes of
    the checkpoint's config; without tokenizer files the tokenizer is None."""
    L, H, D = 2, 2, 64
    cfg = GPTConfig(n_layer=L, n_head=H, n_embd=D, block_size=1024)
    w = R.init_weights(L, H, D, seed=23)
    save_hf_checkpoint(str(tmp_path), w, cfg)
    loader = HFWeightLoader(str(tmp_path))
    sd, tok = loader.load(device=str(gpu))
    assert tok is None and loader.tokenizer is None
    assert loader.config == dict(n_layer=L, n_head=H, n_embd=D)
    expect = internal_to_hf(w, L)
    expect["lm_head.weight"] = expect["transformer.wte.weight"]  # listed, tied
    assert set(sd) == set(expect)
    for k, v in expect.items():
        assert sd[k].is_cuda and torch.equal(sd[k].cpu(), v), k
    assert sd["transformer.h.0.mlp.c_fc.weight"].shape == (D, 4 * D)  # Conv1D (in, out)


def test_pytorch_model_bin_checkpoint(gpu, tmp_path):
    """A directory holding pytorch_model.bin (no safetensors) loads through
    torch.load(weights_only=True) and gives the logits of the safetensors
    directory with the same weights."""
    L, H, D = 2, 4, 128
    cfg = GPTConfig(n_layer=L, n_head=H, n_embd=D, block_size=1024)
    w = R.init_weights(L, H, D, seed=24, dtype=torch.bfloat16)
    st_dir, bin_dir = tmp_path / "st", tmp_path / "bin"
    save_hf_checkpoint(str(st_dir), w, cfg)
    os.makedirs(bin_dir)
    with open(st_dir / "config.json") as f:
        conf = json.load(f)
    with open(bin_dir / "config.json", "w") as f:
        json.dump(conf, f)
    sd = internal_to_hf(w, L)
    sd["lm_head.weight"] = sd["transformer.wte.weight"]
    torch.save(sd, bin_dir / "pytorch_model.bin")
    a = CutileGPT(cfg, dtype=torch.bfloat16, seed=1)
    a.load_from_huggingface(str(bin_dir))
    b = CutileGPT(cfg, dtype=torch.bfloat16, seed=2)
    b.load_from_huggingface(str(st_dir))
    ids = torch.randint(0, 50257, (2, 29), generator=torch.Generator().manual_seed(25)).to(gpu)
    la, lb = a(ids)[0], b(ids)[0]
    assert torch.equal(la, lb)
    exact = R.gpt_forward(w, ids.cpu(), H, R.FLOWS["fp64"])
    assert (la.double().cpu() - exact).abs().max().item() <= 3e-2


def test_bf16_logits_option(gpu):
    """logits_dtype=torch.bfloat16: the LM head rounds the same fp32 accumulators
    to bf16, so the logits are the fp32-logits forward's rounded to bf16, and
    within the bf16 bar of the exact forward."""
    L, H, D = 2, 4, 128
    cfg = GPTConfig(n_layer=L, n_head=H, n_embd=D, block_size=1024)
    w = R.init_weights(L, H, D, seed=26, dtype=torch.bfloat16)
    m32 = CutileGPT(cfg, dtype=torch.bfloat16, seed=0)
    m32.load_weights(w)
    m16 = CutileGPT(cfg, dtype=torch.bfloat16, seed=0, logits_dtype=torch.bfloat16)
    m16.load_weights(w)
    ids = torch.randint(0, 50257, (3, 70), generator=torch.Generator().manual_seed(27)).to(gpu)
    l32, l16 = m32(ids)[0], m16(ids)[0]
    assert l16.dtype == torch.bfloat16 and l16.shape == (3, 70, 50257)
    assert torch.equal(l16, l32.to(torch.bfloat16))
    exact = R.gpt_forward(w, ids.cpu(), H, R.FLOWS["fp64"])
    assert (l16.double().cpu() - exact).abs().max().item() <= 3e-2
