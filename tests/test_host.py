"""Host-side logic on the CPU: the C ABI library, argument validation, config
presets and the HF checkpoint loader.  No kernel is launched here."""

import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cgpt.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(cgpt_\w+)\s*\(", text, re.M)))


def test_library_exports_every_header_symbol():
    from cutilegpt_amd import _lib
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 8
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert lib.cgpt_version() == _lib.ABI_VERSION


def test_status_strings():
    from cutilegpt_amd import _lib
    lib = _lib.load()
    assert lib.cgpt_status_string(0) == b"ok"
    assert b"invalid" in lib.cgpt_status_string(-1)
    assert b"dtype" in lib.cgpt_status_string(-2)
    assert b"shape" in lib.cgpt_status_string(-3)


def test_abi_rejects_bad_arguments_before_launch():
    """Argument errors return negative status without touching the GPU (the
    pointers here are never dereferenced)."""
    from cutilegpt_amd import _lib
    lib = _lib.load()
    fake = 1 << 20  # 16-byte aligned, never dereferenced
    # gemm: A not element-aligned (any K is accepted), bad epilogue, missing bias, bad dtype,
    # fp16 inputs with a bf16 bias / output, lda < K, unknown tile
    assert lib.cgpt_gemm(fake + 1, fake, None, fake, 4, 4, 12, 12, 12, 4, 1, 1, 1, 0, -1, None) == -1
    assert lib.cgpt_gemm(fake, fake, fake, fake, 4, 4, 16, 16, 16, 4, 2, 1, 2, 1, -1, None) == -2
    assert lib.cgpt_gemm(fake, fake, None, fake, 4, 4, 16, 16, 16, 4, 2, 2, 1, 0, -1, None) == -2
    assert lib.cgpt_gemm(fake, fake, None, fake, 4, 4, 16, 16, 16, 4, 1, 1, 1, 7, -1, None) == -1
    assert lib.cgpt_gemm(fake, fake, None, fake, 4, 4, 16, 16, 16, 4, 1, 1, 1, 1, -1, None) == -1
    assert lib.cgpt_gemm(fake, fake + 3, None, fake, 4, 4, 16, 16, 16, 4, 0, 0, 0, 0, -1, None) == -1
    assert lib.cgpt_gemm(fake, fake, None, fake, 4, 4, 16, 16, 16, 4, 5, 1, 1, 0, -1, None) == -2
    assert lib.cgpt_gemm(fake, fake, None, fake, 4, 4, 16, 8, 16, 4, 1, 1, 1, 0, -1, None) == -1
    assert lib.cgpt_gemm(fake, fake, None, fake, 4, 4, 16, 16, 16, 4, 1, 1, 1, 0, 99, None) == -1
    # empty problems are a no-op success
    assert lib.cgpt_gemm(None, None, None, None, 0, 4, 16, 16, 16, 4, 1, 1, 1, 0, -1, None) == 0
    # layernorm (any width): x / y not element-aligned, bad dtype, null gamma, negative eps
    assert lib.cgpt_add_layernorm(fake + 2, None, None, fake, fake, fake, 2, 6, 1e-5, 0, 0, 0, 0, None) == -1
    assert lib.cgpt_add_layernorm(fake, None, None, fake, fake, fake + 1, 2, 6, 1e-5, 2, 0, 2, 2, None) == -1
    assert lib.cgpt_add_layernorm(fake, None, None, fake, fake, fake, 2, 8192, -1.0, 0, 0, 0, 0, None) == -1
    assert lib.cgpt_add_layernorm(fake, None, None, fake, fake, fake, 2, 8, 1e-5, 3, 0, 0, 0, None) == -2
    assert lib.cgpt_add_layernorm(fake, None, None, None, fake, fake, 2, 8, 1e-5, 0, 0, 0, 0, None) == -1
    # attention: unsupported head_dim, Tk < Tq, unaligned strides, bad scale
    args = lambda hd, tq, tk, st, scale: (fake, fake, fake, fake, 1, 1, tq, tk, hd,
                                          *([0, 0, st] * 4), scale, 1, 1, None)
    assert lib.cgpt_attention_fwd(*args(48, 4, 4, 48, 0.1)) == -3
    assert lib.cgpt_attention_fwd(*args(64, 8, 4, 64, 0.1)) == -1
    assert lib.cgpt_attention_fwd(*args(64, 4, 4, 60, 0.1)) == -1
    assert lib.cgpt_attention_fwd(*args(64, 4, 4, 64, 0.0)) == -1
    # gelu / embedding
    assert lib.cgpt_gelu(fake, fake, 10, 9, None) == -2
    assert lib.cgpt_gelu(None, None, 0, 0, None) == 0
    # embedding (any width): wte not element-aligned, fp16 weights into bf16
    assert lib.cgpt_embedding(fake, fake + 2, None, fake, 4, 4, 6, 10, 0, 0, 0, 0, None, None) == -1
    assert lib.cgpt_embedding(fake, fake, None, fake, 4, 4, 6, 10, 0, 0, 2, 1, None, None) == -2
    # embedding + LayerNorm: D not a multiple of 4, missing wpe, bad dtype, misaligned x_out
    el = lambda wpe, x, D, wd: lib.cgpt_embedding_layernorm(fake, fake, wpe, None, x, fake, fake, fake,
                                                             4, 4, D, 10, 0, 8, 1e-5, wd, 0, None, None)
    assert el(fake, fake, 6, 0) == -3
    assert el(None, fake, 8, 0) == -1
    assert el(fake, fake, 8, 4) == -2
    assert el(fake, fake + 4, 8, 0) == -1


def test_wrappers_reject_host_tensors():
    import cutilegpt_amd as cg
    x = torch.randn(4, 8)
    with pytest.raises(ValueError):
        cg.cutile_gelu(x)
    with pytest.raises(ValueError):
        cg.cutile_layer_norm(x, torch.ones(8), torch.zeros(8))
    with pytest.raises(ValueError):
        cg.cutile_linear(x, torch.randn(3, 8))
    with pytest.raises(ValueError):
        cg.cutile_causal_attention(x.view(1, 1, 4, 8), x.view(1, 1, 4, 8), x.view(1, 1, 4, 8), 1)
    with pytest.raises(ValueError):
        cg.cutile_embedding(torch.tensor([1, 2]), x)


def test_config_presets_match_reference():
    from cutilegpt_amd import GPTConfig
    # cutile_gpt/models/config.py:19-87
    expect = {"nano": (3, 3, 48, 128), "micro": (4, 4, 128, 256), "mini": (6, 6, 192, 256),
              "gpt2": (12, 12, 768, 1024), "gpt2-medium": (24, 16, 1024, 1024),
              "gpt2-large": (36, 20, 1280, 1024), "gpt2-xl": (48, 25, 1600, 1024),
              "tile-small": (4, 4, 64, 128), "tile-medium": (6, 4, 128, 256),
              "tile-large": (8, 8, 256, 512)}
    for name, (l, h, d, bs) in expect.items():
        c = GPTConfig.from_name(name)
        assert (c.n_layer, c.n_head, c.n_embd, c.block_size, c.vocab_size) == (l, h, d, bs, 50257)
    with pytest.raises(ValueError):
        GPTConfig.from_name("gpt5")


def test_hf_checkpoint_roundtrip_and_transformers_agree(tmp_path):
    """save_hf_checkpoint writes a directory that transformers itself loads,
    and load_hf_checkpoint maps it back to the internal layout exactly."""
    from cutilegpt_amd.config import GPTConfig
    from cutilegpt_amd.hf_loader import load_hf_checkpoint, save_hf_checkpoint
    from oracle import gpt_ref as R
    from transformers import GPT2LMHeadModel

    cfg = GPTConfig(n_layer=2, n_head=2, n_embd=32, block_size=64, vocab_size=50257)
    # every bias and LayerNorm tensor distinct, as in a trained checkpoint
    w = R.randomize_affine(R.init_weights(2, 2, 32, block_size=64, seed=11), seed=12)
    save_hf_checkpoint(str(tmp_path), w, cfg)
    w2, cfg2 = load_hf_checkpoint(str(tmp_path))
    assert cfg2 == cfg
    for k in w:
        assert torch.equal(w[k], w2[k]), k
    assert w2["lm_head.weight"] is w2["wte"]
    m = GPT2LMHeadModel.from_pretrained(str(tmp_path)).eval()
    ids = torch.randint(0, 50257, (1, 20), generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        ref = m(ids).logits
    out = R.gpt_forward(w2, ids, 2, R.FLOWS["fp32"])
    assert (out - ref).abs().max().item() < 1e-5
    # transformers reads each bias / LayerNorm tensor from the key it was written to
    sd = m.state_dict()
    for i in range(2):
        for name in ("ln_1.weight", "ln_1.bias", "attn.c_attn.bias", "attn.c_proj.bias",
                     "ln_2.weight", "ln_2.bias", "mlp.c_fc.bias", "mlp.c_proj.bias"):
            assert torch.equal(sd[f"transformer.h.{i}.{name}"], w[f"h.{i}.{name}"]), (i, name)


def test_tile_table_lookup():
    from cutilegpt_amd import tiles, _lib
    assert tiles.gemm_tile(_lib.CGPT_BF16, 3, 5, 8) == _lib.TILE_AUTO
    n = _lib.load().cgpt_gemm_num_tiles()
    for key, t in tiles.TABLE.items():
        assert 0 <= t < n, key
        assert tiles.m_bucket(key[1]) == key[1], key  # keys hold bucket values
    # one entry covers every M of its bucket, (bucket / 2, bucket]
    assert tiles.m_bucket(1) == 1 and tiles.m_bucket(4096) == 4096
    assert tiles.m_bucket(4097) == 8192 and tiles.m_bucket(2049) == 4096
    bf = _lib.CGPT_BF16
    assert tiles.gemm_tile(bf, 16384, 2304, 768) == tiles.gemm_tile(bf, 8200, 2304, 768) == 14
    assert tiles.gemm_tile(bf, 8192, 2304, 768) == _lib.TILE_AUTO
    assert tiles.gemm_tile(bf, 3000, 512, 512) == 19


def test_sampling_semantics_temperature_and_top_k():
    """CutileGPT._sample follows cutile_gpt/models/gpt.py:207-226: logits are
    divided by the temperature, everything below the k-th largest is masked,
    and the token is drawn from the softmax of the rest (top_k=1: the argmax).
    Checked by drawing many samples from fixed logits on the CPU: every draw
    lies in the top-k set and the frequencies match softmax(logits / T) over
    that set within 5 standard errors."""
    from cutilegpt_amd.model import CutileGPT
    g = torch.Generator().manual_seed(0)
    base = torch.randn(2, 40, generator=g) * 2.0
    n = 40000
    for temperature, top_k in ((0.7, 5), (1.5, 3), (1.0, None), (0.3, 40)):
        torch.manual_seed(1)
        logits = base.repeat_interleave(n, dim=0)
        tok = CutileGPT._sample(logits, temperature, top_k).view(2, n)
        for r in range(2):
            z = base[r].double() / temperature
            allowed = torch.ones_like(z, dtype=torch.bool)
            if top_k is not None:
                allowed = z >= torch.topk(z, top_k).values[-1]
            p = torch.where(allowed, z, torch.tensor(float("-inf"), dtype=z.dtype)).softmax(-1)
            assert allowed[tok[r]].all(), (temperature, top_k)
            freq = torch.bincount(tok[r], minlength=40).double() / n
            se = (p * (1 - p) / n).sqrt()
            assert ((freq - p).abs() <= 5 * se + 1e-12).all(), (temperature, top_k)
    # top_k = 1 is greedy whatever the temperature; a tiny temperature is too.
    assert torch.equal(CutileGPT._sample(base, 3.0, 1).view(-1), base.argmax(-1))
    assert torch.equal(CutileGPT._sample(base, 1e-6, None).view(-1), base.argmax(-1))


def test_attention_qkv_rejects_host_tensors():
    import cutilegpt_amd as cg
    with pytest.raises(ValueError):
        cg.attention_qkv(torch.zeros(1, 4, 3 * 64, dtype=torch.bfloat16), 2)


def test_tune_shapes_cover_the_table():
    """The sweep's shapes are the forward's GEMMs (c_attn, attn c_proj, c_fc,
    MLP c_proj, padded LM head) per config, and every TABLE entry is one of
    them at its M bucket."""
    from cutilegpt_amd import tune, tiles, _lib
    got = set()
    for name, (d, m) in tune.CONFIGS.items():
        sh = tune.shapes(name)
        assert [s[0] for s in sh] == ["c_attn", "attn_c_proj", "c_fc_gelu", "mlp_c_proj", "lm_head"]
        assert [(s[2], s[3]) for s in sh] == [(3 * d, d), (d, d), (4 * d, d), (d, 4 * d),
                                              (tune.VOCAB_PAD, d)]
        assert sh[1][4] == sh[3][4] == _lib.EPI_BIAS_RESID and sh[2][4] == _lib.EPI_BIAS_GELU
        got |= {(_lib.CGPT_BF16, tiles.m_bucket(s[1]), s[2], s[3]) for s in sh}
    assert set(tiles.TABLE) <= got
