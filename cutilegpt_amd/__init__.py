"""cutilegpt_amd — cutileGPT's GPT-2 forward hot path on MI355X (gfx950).

Drop-in names of the reference package (``cutile_gpt/__init__.py:41-129``):
the ``cutile_*`` kernel functions, ``CutileGPT``, ``GPTConfig`` and
``HFWeightLoader``, implemented with hand-written CDNA4 HIP kernels
(``csrc/*.hip``, C ABI in ``include/cgpt.h``) called through ctypes on
PyTorch-ROCm tensors and streams.
"""

__version__ = "0.1.0"

from .config import GPTConfig  # noqa: F401
from .kernels import (  # noqa: F401
    add_layer_norm,
    attention_qkv,
    cutile_causal_attention,
    cutile_embedding,
    cutile_fused_mlp,
    cutile_gelu,
    cutile_layer_norm,
    cutile_linear,
    cutile_linear_bias,
    linear_bias_gelu,
    token_pos_embedding,
)
from .model import CutileGPT  # noqa: F401
from .hf_loader import HFWeightLoader  # noqa: F401
from . import api  # noqa: F401  (Tile API: cutilegpt_amd.api.tile, configure_tiles, ...)

__all__ = [
    "__version__",
    "CutileGPT",
    "GPTConfig",
    "HFWeightLoader",
    "cutile_gelu",
    "cutile_embedding",
    "cutile_linear",
    "cutile_linear_bias",
    "cutile_layer_norm",
    "cutile_causal_attention",
    "cutile_fused_mlp",
    "add_layer_norm",
    "linear_bias_gelu",
    "attention_qkv",
    "token_pos_embedding",
]
