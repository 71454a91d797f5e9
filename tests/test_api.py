"""Tile API graph building on the CPU: shapes, validation errors, the
linear+GELU fusion pass, TileConfig -> tile-id wiring and DataAnalyzer
statistics (execution is covered by test_api_gpu.py)."""

import numpy as np
import pytest
import torch

from cutilegpt_amd import _lib, api
from cutilegpt_amd.api import (DataAnalyzer, DType, Layout, OpType, TensorSpec, TileConfig, TileOp,
                               configure_tiles, tile)


def x3(b=2, t=8, d=48, dtype=torch.float32):
    return torch.zeros(b, t, d, dtype=dtype)


def test_chain_shapes_and_names():
    w = torch.zeros(192, 48)
    op = (tile(x3(), "h").declare_shape(batch=2, seq=8, dim=48)
          .linear(w, torch.zeros(192), out_features=192).gelu())
    assert op.shape == (2, 8, 192)
    assert op.spec.dim_names == ("batch", "seq", "out_features")
    assert [o.op_type for o in op.ops] == [OpType.INPUT, OpType.LINEAR_BIAS, OpType.GELU]
    assert op.spec.name == "h_linear_gelu"
    text = op.describe()
    assert "LINEAR_BIAS" in text and "Final:" in text and "(2, 8, 192)" in text


def test_linear_without_bias_and_transposed_weight():
    op = tile(x3()).linear(torch.zeros(48, 96), weight_transposed=True)
    assert op.ops[-1].op_type == OpType.LINEAR
    assert op.shape == (2, 8, 96)
    assert op.ops[-1].params["weight_transposed"] is True


def test_validation_errors():
    with pytest.raises(ValueError, match="in_features"):
        tile(x3()).linear(torch.zeros(10, 47))
    with pytest.raises(ValueError, match="out_features"):
        tile(x3()).linear(torch.zeros(10, 48), out_features=11)
    with pytest.raises(ValueError, match="doesn't match"):
        tile(x3()).declare_shape(batch=2, seq=9, dim=48)
    with pytest.raises(ValueError, match="normalized_shape"):
        tile(x3()).layernorm(torch.ones(47), torch.zeros(47))
    with pytest.raises(ValueError, match="hidden_features"):
        tile(x3()).fused_mlp(torch.zeros(192, 48), torch.zeros(192), torch.zeros(48, 192),
                             torch.zeros(48), hidden_features=100)
    with pytest.raises(ValueError):
        TileOp.from_tensor(np.zeros((2, 3)))
    with pytest.raises(ValueError, match="-1"):
        tile(x3()).reshape(-1, -1)
    with pytest.raises(ValueError, match="tanh"):
        tile(x3()).gelu(approximate=False)


def test_attention_spec_from_fused_projection():
    op = tile(x3(d=144)).attention(n_head=3)
    p = op.ops[-1].params
    assert op.shape == (2, 8, 48)
    assert p["head_dim"] == 16 and abs(p["scale"] - 0.25) < 1e-12 and p["causal"]


def test_reshape_transpose_and_mlp_shapes():
    op = tile(x3()).reshape(-1, 48)
    assert op.shape == (16, 48)
    op = tile(x3()).transpose()
    assert op.shape == (2, 48, 8)
    op = tile(x3()).transpose(1, 0, 2)
    assert op.shape == (8, 2, 48)
    op = tile(x3()).fused_mlp(torch.zeros(192, 48), torch.zeros(192), torch.zeros(48, 192),
                              torch.zeros(48))
    assert op.shape == (2, 8, 48) and op.ops[-1].params["hidden_features"] == 192


def test_builder_returns_new_ops():
    base = tile(x3())
    a = base.gelu()
    b = base.layernorm(torch.ones(48), torch.zeros(48))
    assert len(base.ops) == 1 and len(a.ops) == 2 and len(b.ops) == 2


def test_fusion_pass():
    w, b = torch.zeros(96, 48), torch.zeros(96)
    op = tile(x3()).linear(w, b).gelu().linear(torch.zeros(48, 96), torch.zeros(48)).gelu().gelu()
    fused = op._fused_ops()
    kinds = [(o.op_type, o.params.get("gelu", False)) for o in fused]
    assert kinds == [(OpType.INPUT, False), (OpType.LINEAR_BIAS, True),
                     (OpType.LINEAR_BIAS, True), (OpType.GELU, False)]
    # A bias-free linear keeps its GELU separate (no bias epilogue to fuse into).
    op = tile(x3()).linear(w).gelu()
    assert [o.op_type for o in op._fused_ops()] == [OpType.INPUT, OpType.LINEAR, OpType.GELU]
    assert [o.op_type for o in op.ops] == [OpType.INPUT, OpType.LINEAR, OpType.GELU]


def test_tile_config_validation_and_mapping():
    assert TileConfig().gemm_tile(torch.bfloat16) is None
    assert configure_tiles(256, 192).gemm_tile(torch.bfloat16) == 14
    assert configure_tiles(256, 256, 64).gemm_tile(torch.bfloat16) == 12
    assert configure_tiles(128, 64).gemm_tile(torch.bfloat16) == 3
    assert configure_tiles(128, 128).gemm_tile(torch.float32) == 0
    assert configure_tiles(128, 128).gemm_tile(torch.float16) == 2
    assert configure_tiles(256, 192).gemm_tile(torch.float16) == 14
    with pytest.raises(ValueError, match="no"):
        configure_tiles(256, 256).gemm_tile(torch.float32)
    with pytest.raises(ValueError, match="power of 2"):
        TileConfig(tile_m=96)
    with pytest.raises(ValueError, match="power of 2"):
        TileConfig(tile_k=0)
    n = _lib.load().cgpt_gemm_num_tiles()
    for t in list(api._BF16_TILES.values()):
        assert 0 <= t < n


def test_tile_config_travels_with_ops():
    cfg = configure_tiles(128, 64)
    op = tile(x3()).with_tile_config(cfg).linear(torch.zeros(96, 48), torch.zeros(96))
    assert op.ops[-1].tile_config is cfg


def test_tensor_spec():
    s = TensorSpec((2, 3, 4), DType.BFLOAT16, Layout.ROW_MAJOR, "x", ("a", "b", "c"))
    assert s.ndim == 3 and s.numel == 24
    assert s.with_shape(6, 4).shape == (6, 4)
    assert "BFLOAT16" in repr(s)
    assert DType.from_torch(torch.bfloat16) == DType.BFLOAT16
    assert DType.BFLOAT16.to_torch() == torch.bfloat16


def test_placeholder_cannot_execute():
    op = TileOp.placeholder((2, 4), name="p").gelu()
    with pytest.raises(ValueError, match="no input data"):
        op.execute()


def test_data_analyzer():
    prof = DataAnalyzer().analyze([[1, 2, 3], [4, 5], [], np.array([7, 7, 7, 7])], name="d")
    assert prof.source == "list" and prof.sample_count == 4
    assert prof.sequence_lengths == [3, 2, 4]
    assert prof.min_sequence_length == 2 and prof.max_sequence_length == 4
    assert abs(prof.avg_sequence_length - 3.0) < 1e-12
    assert prof.unique_tokens == 6 and prof.vocab_size == 8
    assert 1 <= prof.recommended_batch_size <= 64
    # Without a tokenizer strings map character by character.
    prof = DataAnalyzer().analyze(["ab", "abc"])
    assert prof.unique_tokens == 3 and prof.vocab_size == ord("c") + 1
    # Long sequences at a large batch fill the CUs with 256 x 192 tiles.
    prof = DataAnalyzer().analyze([list(range(1024))] * 4)
    assert (prof.recommended_tile_m, prof.recommended_tile_n) == (256, 192)
    prof = DataAnalyzer().analyze(np.arange(12).reshape(3, 4))
    assert prof.source == "array" and prof.sample_count == 3
