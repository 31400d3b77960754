"""adaLN modulation table (model/fusion.py:68-69): oracle pins (CPU).

The oracle takes the activations a = bf16(silu(temb)) and sums a @ W^T in
the kernel's defined fp32 order. It is pinned by exact integer sums (order
cannot matter), by hand-built rows where the order decides the result, and
against torch's own fp32 linear within a bf16 ulp.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_bf16_close, bf16_randn, to_np
from oracle import bf16, reference as ref


def test_exact_when_no_rounding_happens():
    g = torch.Generator().manual_seed(1)
    a = torch.randint(-8, 9, (3, 5120), generator=g).float()
    w = torch.randint(-8, 9, (96, 5120), generator=g).float()
    bias = torch.randint(-64, 65, (96,), generator=g).float()
    out = ref.adaln_table(to_np(a.bfloat16()), to_np(w.bfloat16()), to_np(bias.bfloat16()))
    exact = (a.double() @ w.double().t() + bias.double()).float()       # |sum| < 2^24: exact
    assert np.array_equal(out, to_np(exact.bfloat16()))


def _row(k, entries):
    a = np.zeros(k, np.float32)
    w = np.zeros(k, np.float32)
    for i, (x, y) in entries.items():
        a[i], w[i] = x, y
    return bf16.from_f32(a[None]), bf16.from_f32(w[None])


@pytest.mark.parametrize("entries,expect", [
    # lane 0 holds chunks 0 and 64, lane 1 chunks 1 and 65, ... (8 elements each).
    # 2^24 in lane 0; ones in lanes 1 and 33 meet first (h = 32) -> 2 survives.
    ({0: (4096.0, 4096.0), 8: (1.0, 1.0), 264: (1.0, 1.0)}, 2.0),
    # ones in lanes 32 and 1: lane 32 meets the 2^24 of lane 0 first -> absorbed one by one.
    ({0: (4096.0, 4096.0), 256: (1.0, 1.0), 8: (1.0, 1.0)}, 0.0),
    # inside lane 0: chunk 0 (the 2^24) comes before chunk 64 (two ones) -> absorbed.
    ({0: (4096.0, 4096.0), 512: (1.0, 1.0), 513: (1.0, 1.0)}, 0.0),
])
def test_summation_order(entries, expect):
    a, w = _row(1024, entries)
    bias = bf16.from_f32(np.array([-(2.0 ** 24)], np.float32))
    out = ref.adaln_table(a, w, bias)
    assert bf16.to_f32(out)[0, 0] == np.float32(expect)


@pytest.mark.parametrize("rows,k,n", [(1, 5120, 384), (6, 5120, 256), (3, 264, 50)])
def test_close_to_torch_linear(rows, k, n):
    g = torch.Generator().manual_seed(rows * 100 + n)
    temb = torch.randn(rows, k, generator=g) * 2
    a = F.silu(temb).to(torch.bfloat16)
    w = bf16_randn((n, k), g, scale=0.02)
    bias = bf16_randn((n,), g, scale=0.1)
    ours = ref.adaln_table(to_np(a), to_np(w), to_np(bias))
    theirs = F.linear(a.float(), w.float(), bias.float()).bfloat16()
    assert_bf16_close(ours, to_np(theirs), max_ulp=1, frac_exact=0.98)
