"""Drop-in for the reference's model/int8_tma.py (`matmul`).

The reference keeps a second, Hopper-only GEMM for long sequences: a
persistent Triton kernel with TMA descriptor loads (model/int8_tma.py:12-41),
chosen by int8_matmul for M >= 16384 on compute capability 9. Its job on
Hopper -- persistent blocks, grouped tile order, bulk loads of whole operand
tiles -- is what the gfx950 GEMM already does for every M: whole-line
global->LDS DMAs, XCD-aware grouped tile order. This module keeps the entry
point, its argument checks and its output, and runs that GEMM.
"""
from __future__ import annotations

import torch

from .int8_gemm import int8_matmul

_REFERENCE_TILE = (128, 256, 128, 8, 3)


def matmul(a, b, sa, sb, bias=None, tile=_REFERENCE_TILE):
    """bf16(((float)(a @ b) * sa) * sb + bias), a int8 [M, K] row-major, b int8
    [K, N] as the transposed view of row-major [N, K] weights (stride (1, K)).

    `tile` keeps the reference's (BM, BN, BK, warps, stages) form; the
    reference's default selects the shape heuristic, any other value the HIP
    tile of that (BM, BN) (ValueError when there is none).
    """
    m, k = a.shape
    if a.dtype != torch.int8 or b.dtype != torch.int8 or not a.is_contiguous() or b.stride() != (1, k):
        raise ValueError("TMA requires row-major INT8 activations and transposed row-major weights")
    return int8_matmul(a, b, sa, sb, bias, tile=None if tuple(tile) == _REFERENCE_TILE else tile)
