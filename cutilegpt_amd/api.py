"""Declarative Tile API on the gfx950 kernels.

Mirrors ``cutile_gpt/api`` (``api/__init__.py:19-55``): ``tile(x)`` starts a
fluent chain (``linear``, ``gelu``, ``layernorm``, ``attention``, ``fused_mlp``,
``reshape``, ``transpose``) that records ``OpNode``s and runs them on
``execute()``; ``TileConfig`` / ``TensorSpec`` / ``Layout`` / ``DType`` /
``configure_tiles`` and the ``DataProfile`` / ``DataAnalyzer`` helpers keep
their names and fields.  Differences, all on purpose:

* Tensors are torch tensors (the reference takes CuPy arrays); anything else
  raises ``ValueError`` as the reference does for non-CuPy input
  (``api/tile_op.py:79-80``).  Execution needs them on the GPU.
* ``TileConfig`` is wired to the GEMM tile table (the reference's is unused):
  the default ``TileConfig()`` keeps the library's tuned choice per problem,
  any other ``(tile_m, tile_n)`` selects the gfx950 tile of that size
  (``TileConfig.gemm_tile``).  Hardware hints written for another GPU
  (``num_ctas``, ``use_tma``, ``use_tf32`` ...) are accepted and ignored.
* ``execute(optimize=True)`` fuses ``linear(w, b)`` followed by ``gelu()`` into
  one GEMM with the GELU in its epilogue (the reference's ``_optimize_graph``
  is a placeholder, ``api/tile_op.py:438-440``), and ``attention`` on a fused
  (B, T, 3D) projection reads Q, K, V in place instead of splitting and
  transposing them (``api/tile_op.py:474-488``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

from . import _lib

# ---------------------------------------------------------------------------
# Configuration (cutile_gpt/api/config.py)


class Layout(Enum):
    """Memory layout of a tensor (``api/config.py:13-17``)."""
    ROW_MAJOR = auto()
    COL_MAJOR = auto()
    TILED = auto()


class DType(Enum):
    """Element types (``api/config.py:20-34``)."""
    FLOAT32 = auto()
    FLOAT16 = auto()
    BFLOAT16 = auto()

    def to_torch(self) -> torch.dtype:
        return {DType.FLOAT32: torch.float32, DType.FLOAT16: torch.float16,
                DType.BFLOAT16: torch.bfloat16}[self]

    @staticmethod
    def from_torch(dtype: torch.dtype) -> "DType":
        return {torch.float32: DType.FLOAT32, torch.float16: DType.FLOAT16,
                torch.bfloat16: DType.BFLOAT16}.get(dtype, DType.FLOAT32)


# (tile_m, tile_n) -> GEMM tile id of libcgpt.so, per input type.  bf16 ids
# name the persistent direct-to-LDS kernels (256-row tiles) and the
# register-staged ones (smaller tiles), for bf16 and fp16 inputs alike; fp32 has
# two register-staged tiles.
_BF16_TILES = {(256, 256): 12, (256, 192): 14, (256, 128): 9, (128, 256): 10,
               (128, 128): 2, (128, 64): 3, (64, 64): 4}
_F32_TILES = {(128, 128): 0, (64, 64): 1}


@dataclass
class TileConfig:
    """Tile configuration (fields of ``api/config.py:37-66``).

    ``tile_m`` / ``tile_n`` pick the GEMM output tile (rows x columns of C);
    the default 64 x 64 x 32 means "the library's tuned choice".  Accepted
    sizes are powers of two and, for the gfx950 256 x 192 tile, 192.
    """
    tile_m: int = 64
    tile_n: int = 64
    tile_k: int = 32
    num_ctas: int = 1
    occupancy: int = 4
    latency_hint: int = 4
    use_tma: bool = True
    use_swizzle: bool = True
    use_tf32: bool = True

    def __post_init__(self):
        for name, val in (("tile_m", self.tile_m), ("tile_n", self.tile_n),
                          ("tile_k", self.tile_k)):
            if val <= 0 or (val & (val - 1) != 0 and val != 192):
                raise ValueError(f"{name}={val} must be power of 2")

    @property
    def is_default(self) -> bool:
        return (self.tile_m, self.tile_n, self.tile_k) == (64, 64, 32)

    def gemm_tile(self, dtype: torch.dtype) -> Optional[int]:
        """Tile id for a GEMM with inputs of ``dtype``; None = library choice."""
        if self.is_default:
            return None
        table = _BF16_TILES if dtype in (torch.bfloat16, torch.float16) else _F32_TILES
        key = (self.tile_m, self.tile_n)
        if key not in table:
            raise ValueError(f"no {dtype} GEMM tile of {key[0]}x{key[1]} on gfx950; "
                             f"available: {sorted(table)}")
        return table[key]


@dataclass
class TensorSpec:
    """Shape, type, layout and dimension names of a tensor (``api/config.py:69-104``)."""
    shape: Tuple[int, ...]
    dtype: DType = DType.FLOAT32
    layout: Layout = Layout.ROW_MAJOR
    name: str = ""
    dim_names: Tuple[str, ...] = ()

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    def with_shape(self, *shape) -> "TensorSpec":
        return TensorSpec(shape=tuple(shape), dtype=self.dtype, layout=self.layout,
                          name=self.name, dim_names=self.dim_names)

    def __repr__(self) -> str:
        dims = f", dims={self.dim_names}" if self.dim_names else ""
        return f"TensorSpec({self.name}: {self.shape}, {self.dtype.name}, {self.layout.name}{dims})"


def configure_tiles(tile_m: int = 64, tile_n: int = 64, tile_k: int = 32, **kwargs) -> TileConfig:
    """``TileConfig(tile_m, tile_n, tile_k, **kwargs)`` (``api/config.py:107-120``)."""
    return TileConfig(tile_m=tile_m, tile_n=tile_n, tile_k=tile_k, **kwargs)


# ---------------------------------------------------------------------------
# Graph (cutile_gpt/api/tile_op.py)


class OpType(Enum):
    """Operation kinds (``api/tile_op.py:27-37``)."""
    INPUT = auto()
    LINEAR = auto()
    LINEAR_BIAS = auto()
    GELU = auto()
    LAYERNORM = auto()
    ATTENTION = auto()
    FUSED_MLP = auto()
    RESHAPE = auto()
    TRANSPOSE = auto()


@dataclass
class OpNode:
    """One recorded operation (``api/tile_op.py:40-50``)."""
    op_type: OpType
    inputs: List[Any] = field(default_factory=list)
    params: Dict[str, Any] = field(default_factory=dict)
    output_spec: Optional[TensorSpec] = None
    tile_config: Optional[TileConfig] = None

    def __repr__(self) -> str:
        return f"OpNode({self.op_type.name}, out={self.output_spec})"


class TileOp:
    """Fluent builder: every method returns a new ``TileOp`` whose op list is
    the old one plus the new node (``api/tile_op.py:53-528``)."""

    def __init__(self, data: Optional[torch.Tensor] = None, spec: Optional[TensorSpec] = None,
                 ops: Optional[List[OpNode]] = None, tile_config: Optional[TileConfig] = None):
        self._data = data
        self._spec = spec
        self._ops: List[OpNode] = ops or []
        self._tile_config = tile_config or TileConfig()
        self._name = spec.name if spec else "tensor"

    # -- construction

    @classmethod
    def from_tensor(cls, tensor: torch.Tensor, name: str = "input",
                    layout: Layout = Layout.ROW_MAJOR) -> "TileOp":
        if not isinstance(tensor, torch.Tensor):
            raise ValueError(f"Expected a torch tensor, got {type(tensor)}")
        spec = TensorSpec(shape=tuple(tensor.shape), dtype=DType.from_torch(tensor.dtype),
                          layout=layout, name=name)
        op = OpNode(op_type=OpType.INPUT, inputs=[tensor], output_spec=spec)
        return cls(data=tensor, spec=spec, ops=[op])

    @classmethod
    def placeholder(cls, shape: tuple, dtype: DType = DType.FLOAT32,
                    name: str = "placeholder") -> "TileOp":
        spec = TensorSpec(shape=tuple(shape), dtype=dtype, name=name)
        return cls(spec=spec, ops=[OpNode(op_type=OpType.INPUT, output_spec=spec)])

    def declare_shape(self, **dims) -> "TileOp":
        expected = tuple(dims.values())
        if self._spec and self._spec.shape != expected:
            raise ValueError(f"Declared shape {expected} doesn't match actual shape "
                             f"{self._spec.shape}")
        if self._spec:
            self._spec = TensorSpec(shape=self._spec.shape, dtype=self._spec.dtype,
                                    layout=self._spec.layout, name=self._spec.name,
                                    dim_names=tuple(dims.keys()))
        return self

    def with_tile_config(self, config: TileConfig) -> "TileOp":
        self._tile_config = config
        return self

    def _then(self, op: OpNode) -> "TileOp":
        return TileOp(data=self._data, spec=op.output_spec, ops=self._ops + [op],
                      tile_config=self._tile_config)

    def _out(self, shape, suffix, dim_names=None) -> TensorSpec:
        return TensorSpec(shape=tuple(shape), dtype=self._spec.dtype, layout=self._spec.layout,
                          name=f"{self._name}_{suffix}",
                          dim_names=self._spec.dim_names if dim_names is None else dim_names)

    # -- operations

    def linear(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
               out_features: Optional[int] = None, weight_transposed: bool = False) -> "TileOp":
        """``y = x W^T (+ b)`` with W (out, in), or (in, out) when ``weight_transposed``."""
        in_features = self._spec.shape[-1]
        actual_out, actual_in = ((weight.shape[1], weight.shape[0]) if weight_transposed
                                 else (weight.shape[0], weight.shape[1]))
        if actual_in != in_features:
            raise ValueError(f"Weight in_features ({actual_in}) doesn't match input dim "
                             f"({in_features})")
        if out_features and out_features != actual_out:
            raise ValueError(f"Declared out_features ({out_features}) doesn't match weight shape "
                             f"({actual_out})")
        names = self._spec.dim_names[:-1] + ("out_features",) if self._spec.dim_names else ()
        op = OpNode(op_type=OpType.LINEAR_BIAS if bias is not None else OpType.LINEAR,
                    inputs=[weight, bias] if bias is not None else [weight],
                    params={"in_features": in_features, "out_features": actual_out,
                            "weight_transposed": weight_transposed},
                    output_spec=self._out(self._spec.shape[:-1] + (actual_out,), "linear", names),
                    tile_config=self._tile_config)
        return self._then(op)

    def gelu(self, approximate: bool = True) -> "TileOp":
        """tanh-approximate GELU (the only form the kernels implement)."""
        if not approximate:
            raise ValueError("gelu(approximate=False) is not implemented: the kernels compute "
                             "the tanh approximation")
        op = OpNode(op_type=OpType.GELU, params={"approximate": approximate},
                    output_spec=self._out(self._spec.shape, "gelu"), tile_config=self._tile_config)
        return self._then(op)

    def layernorm(self, weight: torch.Tensor, bias: torch.Tensor, eps: float = 1e-5,
                  normalized_shape: Optional[tuple] = None) -> "TileOp":
        norm_shape = tuple(normalized_shape or (self._spec.shape[-1],))
        if tuple(weight.shape) != norm_shape:
            raise ValueError(f"Weight shape {tuple(weight.shape)} doesn't match normalized_shape "
                             f"{norm_shape}")
        op = OpNode(op_type=OpType.LAYERNORM, inputs=[weight, bias],
                    params={"eps": eps, "normalized_shape": norm_shape},
                    output_spec=self._out(self._spec.shape, "ln"), tile_config=self._tile_config)
        return self._then(op)

    def attention(self, n_head: int, head_dim: Optional[int] = None, causal: bool = True,
                  scale: Optional[float] = None) -> "TileOp":
        """Causal self-attention.  A last dimension divisible by 3 is read as a
        fused (Q, K, V) projection, as in ``api/tile_op.py:296-307``."""
        n_embd = self._spec.shape[-1]
        fused = n_embd % 3 == 0
        out_embd = n_embd // 3 if fused else n_embd
        if head_dim is None:
            head_dim = out_embd // n_head
        if scale is None:
            scale = 1.0 / math.sqrt(head_dim)
        op = OpNode(op_type=OpType.ATTENTION,
                    params={"n_head": n_head, "head_dim": head_dim, "causal": causal,
                            "scale": scale},
                    output_spec=self._out(self._spec.shape[:-1] + (out_embd,), "attn"),
                    tile_config=self._tile_config)
        return self._then(op)

    def fused_mlp(self, w_fc: torch.Tensor, b_fc: torch.Tensor, w_proj: torch.Tensor,
                  b_proj: torch.Tensor, hidden_features: Optional[int] = None) -> "TileOp":
        in_features = self._spec.shape[-1]
        actual_hidden, out_features = w_fc.shape[0], w_proj.shape[0]
        if hidden_features and hidden_features != actual_hidden:
            raise ValueError(f"Declared hidden_features ({hidden_features}) doesn't match w_fc "
                             f"shape ({actual_hidden})")
        op = OpNode(op_type=OpType.FUSED_MLP, inputs=[w_fc, b_fc, w_proj, b_proj],
                    params={"in_features": in_features, "hidden_features": actual_hidden,
                            "out_features": out_features},
                    output_spec=self._out(self._spec.shape[:-1] + (out_features,), "mlp"),
                    tile_config=self._tile_config)
        return self._then(op)

    def reshape(self, *shape) -> "TileOp":
        new_shape = list(shape)
        neg, known = None, 1
        for i, s in enumerate(new_shape):
            if s == -1:
                if neg is not None:
                    raise ValueError("Only one dimension can be -1")
                neg = i
            else:
                known *= s
        if neg is not None:
            new_shape[neg] = self._spec.numel // known
        op = OpNode(op_type=OpType.RESHAPE, params={"shape": tuple(new_shape)},
                    output_spec=self._out(new_shape, "reshape", ()))
        return self._then(op)

    def transpose(self, *dims) -> "TileOp":
        if not dims:
            n = self._spec.ndim
            dims = tuple(range(n - 2)) + (n - 1, n - 2)
        shape = tuple(self._spec.shape[d] for d in dims)
        names = tuple(self._spec.dim_names[d] for d in dims) if self._spec.dim_names else ()
        op = OpNode(op_type=OpType.TRANSPOSE, params={"dims": tuple(dims)},
                    output_spec=self._out(shape, "transpose", names))
        return self._then(op)

    # -- execution

    def execute(self, optimize: bool = True) -> torch.Tensor:
        """Run the recorded operations on the GPU kernels."""
        ops = self._fused_ops() if optimize else self._ops
        return self._execute_ops(ops)

    def _fused_ops(self) -> List[OpNode]:
        """``LINEAR_BIAS`` directly followed by ``GELU`` becomes one node whose
        GEMM applies the GELU in its epilogue."""
        out: List[OpNode] = []
        for op in self._ops:
            if (op.op_type == OpType.GELU and out and out[-1].op_type == OpType.LINEAR_BIAS
                    and not out[-1].params.get("gelu")):
                prev = out[-1]
                out[-1] = OpNode(op_type=OpType.LINEAR_BIAS, inputs=prev.inputs,
                                 params={**prev.params, "gelu": True},
                                 output_spec=op.output_spec, tile_config=prev.tile_config)
            else:
                out.append(op)
        return out

    def _execute_ops(self, ops: Optional[List[OpNode]] = None) -> torch.Tensor:
        from .kernels import _gemm, attention_qkv, cutile_fused_mlp, cutile_gelu, cutile_layer_norm

        current = self._data
        for op in (self._ops if ops is None else ops):
            t = op.op_type
            if t == OpType.INPUT:
                if op.inputs:
                    current = op.inputs[0]
                continue
            if current is None:
                raise ValueError("TileOp.execute: the graph has no input data (placeholder)")
            if t in (OpType.LINEAR, OpType.LINEAR_BIAS):
                weight = op.inputs[0]
                if op.params.get("weight_transposed"):
                    weight = weight.t().contiguous()
                bias = op.inputs[1] if t == OpType.LINEAR_BIAS else None
                epi = (_lib.EPI_BIAS_GELU if op.params.get("gelu") else
                       _lib.EPI_BIAS if bias is not None else _lib.EPI_NONE)
                tile = (op.tile_config or TileConfig()).gemm_tile(current.dtype)
                current = _gemm(current, weight, bias, epi, None, "TileOp.linear", tile=tile)
            elif t == OpType.GELU:
                current = cutile_gelu(current)
            elif t == OpType.LAYERNORM:
                w, b = op.inputs
                current = cutile_layer_norm(current, w, b, op.params.get("eps", 1e-5))
            elif t == OpType.ATTENTION:
                current = self._attention(current, op.params, attention_qkv)
            elif t == OpType.FUSED_MLP:
                current = cutile_fused_mlp(current, *op.inputs)
            elif t == OpType.RESHAPE:
                current = current.reshape(op.params["shape"])
            elif t == OpType.TRANSPOSE:
                current = current.permute(*op.params["dims"])
        return current

    @staticmethod
    def _attention(x: torch.Tensor, params: Dict[str, Any], attention_qkv):
        n_head, hd = params["n_head"], params["head_dim"]
        if not params.get("causal", True):
            raise ValueError("TileOp.attention: only causal attention is implemented")
        if abs(params["scale"] - 1.0 / math.sqrt(hd)) > 1e-12:
            raise ValueError("TileOp.attention: the kernels use scale = 1/sqrt(head_dim)")
        if x.dim() != 3:
            raise ValueError("TileOp.attention expects (batch, seq, features)")
        B, T, F = x.shape
        if F % 3 != 0 or F // 3 != n_head * hd:
            raise ValueError(f"TileOp.attention: expects a fused (Q, K, V) projection of "
                             f"3 * n_head * head_dim = {3 * n_head * hd} features, got {F}")
        return attention_qkv(x.contiguous(), n_head)

    # -- introspection

    @property
    def spec(self) -> TensorSpec:
        return self._spec

    @property
    def shape(self) -> tuple:
        return self._spec.shape if self._spec else ()

    @property
    def ops(self) -> List[OpNode]:
        return list(self._ops)

    def describe(self) -> str:
        """Readable listing of the recorded graph (``api/tile_op.py:508-525``)."""
        lines = ["TileOp Computation Graph:", "=" * 40]
        for i, op in enumerate(self._ops):
            lines.append(f"{'→' if i else ' '} [{i}] {op.op_type.name}")
            if op.output_spec:
                lines.append(f"      Output: {op.output_spec.shape}")
            for k, v in op.params.items():
                lines.append(f"      {k}: {v}")
        if self._spec:
            lines += ["=" * 40, f"Final: {self._spec}"]
        return "\n".join(lines)

    def __repr__(self) -> str:
        return f"TileOp({self._spec})"


def tile(tensor: torch.Tensor, name: str = "input") -> TileOp:
    """``TileOp.from_tensor(tensor, name)`` (``api/tile_op.py:531-534``)."""
    return TileOp.from_tensor(tensor, name=name)


# ---------------------------------------------------------------------------
# Data profiling (cutile_gpt/api/profiler.py)


@dataclass
class DataProfile:
    """Token-sequence statistics and the tile recommendation derived from them
    (fields of ``api/profiler.py:13-42``)."""
    name: str = ""
    source: str = ""
    sample_count: int = 0
    sequence_lengths: List[int] = field(default_factory=list)
    avg_sequence_length: float = 0.0
    max_sequence_length: int = 0
    min_sequence_length: int = 0
    vocab_size: int = 0
    unique_tokens: int = 0
    token_distribution: Dict[int, int] = field(default_factory=dict)
    recommended_tile_m: int = 64
    recommended_tile_n: int = 64
    recommended_batch_size: int = 1
    estimated_memory_mb: float = 0.0


# HBM of one MI355X and the GPT-2 width the recommendation is sized for.
_HBM_MB = 288 * 1024
_REF_EMBD = 768


class DataAnalyzer:
    """Sequence statistics of a dataset and a gfx950 tile recommendation
    (``api/profiler.py:64-195``; strings are tokenized with ``tokenizer`` or,
    without one, mapped character by character as the reference does)."""

    def __init__(self, tokenizer=None):
        self.tokenizer = tokenizer

    def analyze(self, data: Any, name: str = "dataset", max_samples: int = 1000) -> DataProfile:
        profile = DataProfile(name=name)
        if "Dataset" in type(data).__name__:
            profile.source = "huggingface"
            samples = self._extract_hf_samples(data, max_samples)
        elif isinstance(data, list):
            profile.source = "list"
            samples = data[:max_samples]
        elif isinstance(data, np.ndarray):
            profile.source = "array"
            samples = [data] if data.ndim == 1 else list(data)
        else:
            profile.source = "custom"
            samples = list(data)[:max_samples]
        toks = self._ensure_tokenized(samples)
        profile.sample_count = len(toks)
        profile.sequence_lengths = [len(s) for s in toks if len(s) > 0]
        if profile.sequence_lengths:
            profile.avg_sequence_length = float(np.mean(profile.sequence_lengths))
            profile.max_sequence_length = max(profile.sequence_lengths)
            profile.min_sequence_length = min(profile.sequence_lengths)
        all_tokens = [int(t) for s in toks for t in s]
        profile.unique_tokens = len(set(all_tokens))
        if self.tokenizer is not None:
            profile.vocab_size = getattr(self.tokenizer, "vocab_size", None) or len(self.tokenizer)
        else:
            profile.vocab_size = max(all_tokens) + 1 if all_tokens else 50257
        return self._compute_recommendations(profile)

    @staticmethod
    def _extract_hf_samples(dataset, max_samples: int) -> List:
        samples = []
        for i, item in enumerate(dataset):
            if i >= max_samples:
                break
            for key in ("text", "content", "input_ids"):
                if key in item:
                    samples.append(item[key])
                    break
            else:
                for v in item.values():
                    if isinstance(v, str):
                        samples.append(v)
                        break
        return samples

    def _ensure_tokenized(self, samples: List) -> List[List[int]]:
        out = []
        for s in samples:
            if isinstance(s, str):
                out.append(self.tokenizer.encode(s) if self.tokenizer is not None
                           else [ord(c) % 50257 for c in s])
            elif isinstance(s, (list, tuple, np.ndarray)):
                out.append([int(t) for t in s])
            else:
                out.append([int(s)])
        return out

    def _compute_recommendations(self, profile: DataProfile) -> DataProfile:
        """Batch = max-length sequences whose activations (50 fp32 rows of
        width 768 per token, the reference's estimate) fit one MI355X's HBM,
        capped at 64; tile = the GEMM tile the library picks for the GPT-2 MLP
        up-projection at that token count: 256 x 192 once the grid of such
        tiles fills the 256 CUs, else 128 x 64."""
        max_len = max(profile.max_sequence_length, 1)
        per_sample_mb = max_len * _REF_EMBD * 4 / (1024 * 1024)
        batch = int(_HBM_MB / (per_sample_mb * 50))
        profile.recommended_batch_size = max(1, min(batch, 64))
        rows = profile.recommended_batch_size * max_len
        tiles_256 = ((rows + 255) // 256) * ((4 * _REF_EMBD + 191) // 192)
        if tiles_256 >= 256:
            profile.recommended_tile_m, profile.recommended_tile_n = 256, 192
        else:
            profile.recommended_tile_m, profile.recommended_tile_n = 128, 64
        profile.estimated_memory_mb = per_sample_mb * profile.recommended_batch_size * 10
        return profile


__all__ = ["TileConfig", "TensorSpec", "Layout", "DType", "configure_tiles", "TileOp", "OpType",
           "OpNode", "tile", "DataProfile", "DataAnalyzer"]
