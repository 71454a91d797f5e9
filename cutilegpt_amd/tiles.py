"""gfx950 tile/occupancy table for the GEMM kernel.

Replaces the reference's tile planner — the per-wrapper tile constants
(``cutile_gpt/kernels/linear.py:148-152,208-212``: 32x32x32 for everything but
fp16) and the unwired ``TileConfig`` (``cutile_gpt/api/config.py:36-64``).

Tile ids index the configuration table compiled into libcgpt.so
(``csrc/gemm.hip``):

    bf16: 0 = 256x256 (4 waves, 128x128 each), 1 = 256x128, 2 = 128x128,
          3 = 128x64, 4 = 64x64
    fp32: 0 = 128x128, 1 = 64x64

``TABLE`` maps exact (dtype, M, N, K) problems measured on MI355X to the tile
that won; anything else falls back to the library's own heuristic
(``TILE_AUTO``: the largest tile whose grid fills the 256 CUs).
"""

from __future__ import annotations

from typing import Dict, Tuple

from . import _lib

# (dtype code, M, N, K) -> tile id.  Filled from rocprofv3 sweeps on MI355X.
TABLE: Dict[Tuple[int, int, int, int], int] = {}


def gemm_tile(dtype_code: int, m: int, n: int, k: int) -> int:
    """Tile id for a GEMM problem (exact table hit, else the library heuristic)."""
    return TABLE.get((dtype_code, m, n, k), _lib.TILE_AUTO)
