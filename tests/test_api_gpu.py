"""Tile API execution on the GPU against fp64 references of the same chains
(oracle restatements of the reference kernels)."""

import math

import pytest
import torch

from cutilegpt_amd.api import OpType, configure_tiles, tile
from oracle import gpt_ref as R

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16


def randn(*shape, seed=0, scale=1.0, dtype=F32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def max_err(out, ref):
    return (out.detach().cpu().double() - ref.double()).abs().max().item()


def lin(x, w, b=None):
    y = x.double() @ w.double().t()
    return y if b is None else y + b.double()


@pytest.mark.parametrize("dtype", [F32, BF16, torch.float16])
def test_linear_gelu_chain_fused_and_unfused(gpu, dtype):
    x = randn(2, 40, 64, seed=1, dtype=dtype)
    w = randn(192, 64, seed=2, scale=0.1, dtype=dtype)
    b = randn(192, seed=3, scale=0.1, dtype=dtype)
    ref = R.gelu_tanh(lin(x, w, b))
    op = tile(x.to(gpu)).linear(w.to(gpu), b.to(gpu)).gelu()
    fused = op.execute()
    plain = op.execute(optimize=False)
    assert fused.shape == plain.shape == (2, 40, 192)
    tol = {F32: 1e-5, BF16: 3e-2, torch.float16: 4e-3}[dtype]
    assert max_err(fused, ref) < tol
    assert max_err(plain, ref) < tol


def test_linear_transposed_weight_and_no_bias(gpu):
    x = randn(3, 17, 64, seed=4)
    w = randn(96, 64, seed=5, scale=0.1)
    out = tile(x.to(gpu)).linear(w.t().contiguous().to(gpu), weight_transposed=True).execute()
    assert max_err(out, lin(x, w)) < 1e-5


@pytest.mark.parametrize("cfg", [(256, 192, 64), (256, 256, 64), (128, 64, 32), (64, 64, 64)])
def test_explicit_tile_configs_agree(gpu, cfg):
    """Every wired (tile_m, tile_n) gives the reference result (bf16, K % 64 == 0)."""
    x = randn(4, 150, 128, seed=6, dtype=BF16)
    w = randn(520, 128, seed=7, scale=0.05, dtype=BF16)
    b = randn(520, seed=8, scale=0.1, dtype=BF16)
    op = (tile(x.to(gpu)).with_tile_config(configure_tiles(*cfg))
          .linear(w.to(gpu), b.to(gpu)))
    assert op.ops[-1].tile_config.gemm_tile(BF16) is not None
    out = op.execute()
    assert max_err(out, lin(x, w, b)) < 2e-2


@pytest.mark.parametrize("cfg", [(128, 128, 64), (64, 64, 32)])
def test_fp16_tile_configs(gpu, cfg):
    """fp16 through the Tile API with an explicit tile (the reference's fp16
    default is 128x128x64, ``kernels/linear.py:208-212``)."""
    f16 = torch.float16
    x = randn(4, 150, 136, seed=9, dtype=f16)
    w = randn(264, 136, seed=10, scale=0.05, dtype=f16)
    b = randn(264, seed=11, scale=0.1, dtype=f16)
    op = (tile(x.to(gpu)).with_tile_config(configure_tiles(*cfg))
          .linear(w.to(gpu), b.to(gpu)))
    out = op.execute()
    assert out.dtype == f16
    assert max_err(out, lin(x, w, b)) < 4e-3


def test_layernorm_and_attention_chain(gpu):
    """ln -> fused QKV projection -> attention, as one transformer sub-block."""
    B, T, D, H = 2, 48, 64, 4
    x = randn(B, T, D, seed=9)
    g, beta = 1 + randn(D, seed=10, scale=0.1), randn(D, seed=11, scale=0.1)
    w, b = randn(3 * D, D, seed=12, scale=0.1), randn(3 * D, seed=13, scale=0.1)
    out = (tile(x.to(gpu)).layernorm(g.to(gpu), beta.to(gpu)).linear(w.to(gpu), b.to(gpu))
           .attention(n_head=H).execute())
    h = R.layer_norm(x.double(), g.double(), beta.double(), 1e-5)
    qkv = lin(h, w, b)
    q, k, v = (qkv[..., i * D:(i + 1) * D].view(B, T, H, D // H).transpose(1, 2) for i in range(3))
    ref = R.causal_attention(q, k, v).transpose(1, 2).reshape(B, T, D)
    assert out.shape == (B, T, D)
    assert max_err(out, ref) < 2e-5


def test_fused_mlp_reshape_transpose(gpu):
    x = randn(2, 32, 64, seed=14)
    wf, bf = randn(256, 64, seed=15, scale=0.1), randn(256, seed=16, scale=0.1)
    wp, bp = randn(64, 256, seed=17, scale=0.1), randn(64, seed=18, scale=0.1)
    op = tile(x.to(gpu)).fused_mlp(wf.to(gpu), bf.to(gpu), wp.to(gpu), bp.to(gpu))
    op = op.reshape(-1, 64).transpose()
    assert [o.op_type for o in op.ops][-2:] == [OpType.RESHAPE, OpType.TRANSPOSE]
    out = op.execute()
    ref = lin(R.gelu_tanh(lin(x, wf, bf)), wp, bp).reshape(-1, 64).t()
    assert out.shape == (64, 64)
    assert max_err(out, ref) < 2e-5


def test_attention_rejects_unfused_input(gpu):
    x = randn(1, 8, 64).to(gpu)
    with pytest.raises(ValueError, match="fused"):
        tile(x).attention(n_head=4).execute()
