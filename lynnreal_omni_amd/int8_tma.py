"""Drop-in for the reference's model/int8_tma.py (`matmul`).

The reference keeps a second, Hopper-only GEMM for long sequences: a
persistent Triton kernel with TMA descriptor loads (model/int8_tma.py:12-41),
chosen by int8_matmul for M >= 16384 on compute capability 9. Here the entry
point runs the gfx950 GEMM's persistent variant: one workgroup per CU loops
over the 256x256 tiles in the same XCD-grouped order that the one-tile-per-
workgroup launch deals out (the reference's tl.range(pid, tiles, SMS) loop),
with the same ping-pong k-loop and whole-line global->LDS DMAs, so the output
is bit for bit int8_matmul's. Where the async TMA loads let the reference's
next tile start early, here a tile's last k-steps already load the next
tile's first two k-steps into the LDS rings, and the epilogue stages its
outputs through the one ring slot left free. int8_matmul takes the same
kernel by itself for 256x256 launches of at least two waves of tiles with the
bf16 or GELU epilogue, and one tile per workgroup otherwise.
"""
from __future__ import annotations

import torch

from .int8_gemm import int8_matmul

_REFERENCE_TILE = (128, 256, 128, 8, 3)


def matmul(a, b, sa, sb, bias=None, tile=_REFERENCE_TILE):
    """bf16(((float)(a @ b) * sa) * sb + bias), a int8 [M, K] row-major, b int8
    [K, N] as the transposed view of row-major [N, K] weights (stride (1, K)).

    `tile` keeps the reference's (BM, BN, BK, warps, stages) form; the
    reference's default runs the persistent 256x256 GEMM, any other value the
    HIP tile of that (BM, BN) (ValueError when there is none).
    """
    m, k = a.shape
    if a.dtype != torch.int8 or b.dtype != torch.int8 or not a.is_contiguous() or b.stride() != (1, k):
        raise ValueError("TMA requires row-major INT8 activations and transposed row-major weights")
    return int8_matmul(a, b, sa, sb, bias, tile="persistent" if tuple(tile) == _REFERENCE_TILE else tile)
