"""Drop-in for the reference's model/int8_tma.py (`matmul`).

The reference keeps a second, Hopper-only GEMM for long sequences: a
persistent Triton kernel with TMA descriptor loads (model/int8_tma.py:12-41),
chosen by int8_matmul for M >= 16384 on compute capability 9. Here the entry
point runs the gfx950 GEMM's persistent variant: one workgroup per CU loops
over the 256x256 tiles in the same XCD-grouped order that the one-tile-per-
workgroup launch deals out (the reference's tl.range(pid, tiles, SMS) loop),
with the same k-loop, whole-line global->LDS DMAs and epilogue, so the
output is bit for bit int8_matmul's. int8_matmul itself keeps one tile per
workgroup for every M: the persistent grid measured slower on this chip
(vmcnt counts a tile's output stores, so the next tile's first operand wait
also waits for them).
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
