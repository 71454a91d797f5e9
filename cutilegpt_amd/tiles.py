"""gfx950 tile/occupancy table for the GEMM kernel.

Replaces the reference's tile planner — the per-wrapper tile constants
(``cutile_gpt/kernels/linear.py:148-152,208-212``: 32x32x32 for everything but
fp16) and the unwired ``TileConfig`` (``cutile_gpt/api/config.py:36-64``).

Tile ids index the configuration table compiled into libcgpt.so
(``csrc/gemm.hip``):

    bf16, register-staged double buffer (any K % 8):
          0 = 256x256 (4 waves, 128x128 each), 1 = 256x128, 2 = 128x128,
          3 = 128x64, 4 = 64x64
    bf16, persistent direct-to-LDS pipeline, 8 waves (K % (32 * slabs) == 0):
          5 = 256x256, 2 stages of 2 k32 slabs     6 = 256x256, 4 stages of 1
          7 = 256x192, 2 stages of 2 (128x48/wave) 8 = 256x192 (64x96/wave), 2 of 2
          9 = 256x128, 3 stages of 2               10 = 128x256, 3 stages of 2
          11 = 256x128, 6 stages of 1
    bf16, the same pipeline with A fetched two steps ahead (3 A buffers,
    2 W buffers, 2 k32 slabs per stage; buffer-store outputs only):
          12 = 256x256                             13 = 256x192
    bf16, 2 stages of 2 slabs with each slab's fragment reads issued while the
    previous slab's MFMAs run, output rows staged through LDS and stored as
    whole lines with non-temporal stores (rows of 16-byte multiples;
    otherwise the 2-stage kernel):
          14 = 256x192 (8 waves of 128x48)
    bf16, the 2-stage 256x256 pipeline with each wave's output rows staged
    through its own LDS slot and stored as whole lines:
          15 = 256x256 (8 waves of 128x64)
          16 = the same with non-temporal stores (the LM heads' fp32 logits,
               c_fc + GELU)
    fp32: 0 = 128x128, 1 = 64x64

``TABLE`` maps exact (dtype, M, N, K) problems measured on MI355X to the tile
that won; anything else falls back to the library's own heuristic
(``TILE_AUTO``: the persistent tile that fills the 256 CUs best, else the
register-staged kernel's largest tile giving every CU about two blocks).
"""

from __future__ import annotations

from typing import Dict, Tuple

from . import _lib

# (dtype code, M, N, K) -> tile id.  Winners of an event-timed sweep of every
# tile on MI355X (bias epilogue, bf16 out); TFLOP/s of the winner in comments.
_B = _lib.CGPT_BF16
TABLE: Dict[Tuple[int, int, int, int], int] = {
    # GPT-2 124M prefill, M = 16 x 1024
    (_B, 16384, 2304, 768): 14,   # c_attn       981
    (_B, 16384, 768, 768): 14,    # attn c_proj  841
    (_B, 16384, 3072, 768): 16,   # c_fc + GELU   947 in the forward (858 on id 15)
    (_B, 16384, 768, 3072): 14,   # mlp c_proj  1202
    (_B, 16384, 50304, 768): 16,  # lm head (vocab padded), fp32 out 963
    # 'medium' (8L, d 512) prefill, M = 16 x 256
    (_B, 4096, 1536, 512): 14,    # 431
    (_B, 4096, 2048, 512): 10,    # 520 (GELU epilogue)
    (_B, 4096, 512, 2048): 4,     # 361
    (_B, 4096, 50304, 512): 16,   # lm head (vocab padded), fp32 out
}


def gemm_tile(dtype_code: int, m: int, n: int, k: int) -> int:
    """Tile id for a GEMM problem (exact table hit, else the library heuristic)."""
    return TABLE.get((dtype_code, m, n, k), _lib.TILE_AUTO)
