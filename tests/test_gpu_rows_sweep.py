"""A seeded sweep of the HBM-bound row kernels over odd shapes against the
oracle: the quantizer (model/int8.py:66-67), the fused norm + modulate (+ quant)
and residual variants (model/kernels.py:48-128, :405-419) and the gated residual
(:131-153). Widths cover the register-resident kernels (multiples of 8 up to
8192), the one-row-per-block kernels and element-wise tails; row counts cover
partial persistent slices; tables have one to six rows with random indices.
All outputs bit-exact."""
import numpy as np
import pytest
import torch

import gpu_adapter as gpu
from helpers import bf16_randn, to_np
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _widths(rng, count):
    out = []
    for i in range(count):
        if i % 4 == 3:
            out.append(int(rng.integers(1, 600)))            # any width: element-wise tails
        else:
            out.append(int(rng.integers(1, 1025)) * 8)       # 8 .. 8192, multiples of 8
    return out


def _cases(count=16, seed=20261203):
    rng = np.random.default_rng(seed)
    widths = _widths(rng, count)
    return [(int(rng.integers(1, 900)), w, int(rng.integers(1, 7)), i % 2 == 0)
            for i, w in enumerate(widths)]


def _inputs(t, d, rows, seed):
    g = torch.Generator().manual_seed(seed)
    x = bf16_randn((1, t, d), g, outliers=0.01)
    u = bf16_randn((1, t, d), g)
    w = (1 + 0.05 * torch.randn(d, generator=g)).bfloat16()
    table = bf16_randn((rows, 6 * d), g, scale=0.1)
    idx = torch.randint(0, rows, (t,), generator=g)
    return to_np(x), to_np(u), to_np(w), to_np(table), idx.numpy()


@pytest.mark.parametrize("t,d,rows,sorted_idx", _cases(), ids=str)
def test_norm_family(t, d, rows, sorted_idx):
    x, u, w, table, idx = _inputs(t, d, rows, t * 7919 + d)
    if sorted_idx:          # per-frame layout: runs of equal table rows
        idx = np.sort(idx)
    y = gpu.rms_adaln(x, w, table, idx, 3, 4, 1e-6)
    assert np.array_equal(y, ref.rms_adaln(x, w, table, idx, 3, 4, 1e-6))
    q, s = gpu.rms_adaln_quant(x, w, table, idx, 0, 1, 1e-6)
    rq, rs = ref.rms_adaln_quant(x, w, table, idx, 0, 1, 1e-6)
    assert np.array_equal(q, rq) and np.array_equal(s, rs)
    r, q, s = gpu.residual_rms_quant(x, u, w, table, idx, 1e-6)
    rr, rq, rs = ref.residual_rms_quant(x, u, w, table, idx, 1e-6)
    assert np.array_equal(r, rr) and np.array_equal(q, rq) and np.array_equal(s, rs)
    g = gpu.gated_residual(x, u, table, idx, 5)
    assert np.array_equal(g, ref.gated_residual(x, u, table, idx, 5))


@pytest.mark.parametrize("rows,width", [(int(r), int(w)) for r, w in zip(
    np.random.default_rng(20261204).integers(1, 600, 12),
    np.random.default_rng(20261205).integers(1, 24000, 12))], ids=str)
def test_quantize_rows_any_width(rows, width):
    g = torch.Generator().manual_seed(rows * 31 + width)
    x = bf16_randn((rows, width), g, outliers=0.01)
    q, s = gpu.quantize_rows(to_np(x))
    rq, rs = ref.quantize_rows(to_np(x))
    assert np.array_equal(q, rq)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))
