"""gfx950 tile/occupancy table for the GEMM kernel.

Replaces the reference's tile planner — the per-wrapper tile constants
(``cutile_gpt/kernels/linear.py:148-152,208-212``: 32x32x32 for everything but
fp16) and the unwired ``TileConfig`` (``cutile_gpt/api/config.py:36-64``).

Tile ids index the configuration table compiled into libcgpt.so
(``csrc/gemm.hip``):

    bf16 (every id below also runs fp16 inputs on the fp16 MFMA), register-staged
    double buffer (any K % 8; other K, strides or alignments take the 64x64 tile
    with element loads):
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
    bf16, the 2-3 stage pipeline with 4 waves on small tiles (also with the
    residual epilogue; problems whose 256x192 tiles would leave CUs idle),
    launched with as many blocks as fit a CU (two, or three at 64x64):
          17 = 128x128 (2 stages)  18 = 128x64 (3 stages)  19 = 64x64 (3 stages)
    fp32: 0 = 128x128, 1 = 64x64

``TABLE`` maps (dtype, M bucket, N, K) to the tile that won a sweep of every
tile on MI355X (``python -m cutilegpt_amd.tune``: each model's prefill GEMMs,
bias / GELU / residual epilogues and output types as the forward runs them).
The M bucket is the power of two at or above M, so one entry covers every M
in (bucket / 2, bucket] — batch x sequence products that differ a little share
a choice.  Anything else falls back to the library's own heuristic
(``TILE_AUTO``: the persistent tile that fills the 256 CUs best, else the
register-staged kernel's largest tile giving every CU about two blocks).  For
the residual epilogue (attn / MLP c_proj into the fp32 residual stream) a
tile id picks between the slab kernel (14), the small pipeline tiles (17-19)
and the register-staged tiles.
"""

from __future__ import annotations

from typing import Dict, Tuple

from . import _lib


def m_bucket(m: int) -> int:
    """The power of two at or above ``m`` (1 for m <= 1)."""
    return 1 << max(0, (int(m) - 1).bit_length())


# (dtype code, M bucket, N, K) -> tile id, from the sweep (TFLOP/s by kernel time of the
# winner, inputs hot; attn/MLP c_proj with the residual epilogue, fp32 out).
_B = _lib.CGPT_BF16
TABLE: Dict[Tuple[int, int, int, int], int] = {
    # GPT-2 124M prefill, M = 16 x 1024
    (_B, 16384, 2304, 768): 14,   # c_attn       1075
    (_B, 16384, 768, 768): 14,    # attn c_proj   636
    (_B, 16384, 3072, 768): 16,   # c_fc + GELU  1074
    (_B, 16384, 768, 3072): 14,   # mlp c_proj   1056
    (_B, 16384, 50304, 768): 16,  # lm head (vocab padded), fp32 out  1015
    # 'medium' (8 layers, d 512) prefill, M = 16 x 256
    (_B, 4096, 1536, 512): 14,    # c_attn        474
    (_B, 4096, 512, 512): 19,     # attn c_proj   266 (64x64 pipeline)
    (_B, 4096, 2048, 512): 17,    # c_fc + GELU   580 (128x128 pipeline)
    (_B, 4096, 512, 2048): 19,    # mlp c_proj    497 (64x64 pipeline)
    (_B, 4096, 50304, 512): 16,   # lm head       877
    # GPT-2 XL (48 layers, d 1600) prefill inside generate, M = 32 x 128
    (_B, 4096, 4800, 1600): 14,   # c_attn       1015
    (_B, 4096, 1600, 1600): 17,   # attn c_proj   661 (128x128 pipeline; slab: 144 tiles)
    (_B, 4096, 6400, 1600): 16,   # c_fc + GELU   997 (128x128 pipeline 968)
    (_B, 4096, 1600, 6400): 17,   # mlp c_proj    934 (128x128 pipeline)
    (_B, 4096, 50304, 1600): 16,  # lm head      1156
}


def gemm_tile(dtype_code: int, m: int, n: int, k: int) -> int:
    """Tile id for a GEMM problem (table hit for M's bucket, else the library
    heuristic).  fp16 inputs run the bf16 kernels on the fp16 MFMA at the same
    rate, so they share the bf16 entries."""
    if dtype_code == _lib.CGPT_F16:
        dtype_code = _lib.CGPT_BF16
    return TABLE.get((dtype_code, m_bucket(m), n, k), _lib.TILE_AUTO)
