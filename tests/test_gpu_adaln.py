"""GPU parity of the adaLN table kernel (model/fusion.py:68-69) through the C ABI.

Bit-exact vs the oracle given the activations torch itself computes on the
GPU (F.silu(temb).to(bf16), the reference's expression on this device), so
the fused silu is pinned against torch's and the sum against the defined
order; within a bf16 ulp of torch's own bf16 linear (hipBLASLt) away from
outputs that cancel to near zero."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_bf16_close, bf16_randn, to_np
from lynnreal_omni_amd import kernels
from oracle import reference as ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,k,n,dtype,bias", [
    (1, 5120, 6 * 5120, torch.float32, True),      # one time embedding, the C2 table
    (6, 5120, 6 * 5120, torch.float32, True),      # per-frame times (C5: 6 table rows)
    (2, 5120, 3000, torch.bfloat16, False),
    (11, 1024, 384, torch.float32, True),          # two row groups (8 + 3)
    (3, 264, 50, torch.float32, True),             # K not a multiple of 512: partial chunk sweep
    (8, 8192, 96, torch.bfloat16, True),           # 128 KB of LDS
])
def test_adaln_table_bit_exact(rows, k, n, dtype, bias):
    g = torch.Generator().manual_seed(rows + k + n)
    temb = (torch.randn(rows, k, generator=g) * 3).to(dtype).cuda()
    w = bf16_randn((n, k), g, scale=0.02).cuda()
    b = bf16_randn((n,), g, scale=0.1).cuda() if bias else None
    out = kernels.adaln_table(temb, w, b)
    a = F.silu(temb).to(torch.bfloat16)
    want = ref.adaln_table(to_np(a), to_np(w), None if b is None else to_np(b))
    assert np.array_equal(to_np(out), want)
    # torch's bf16 linear sums in another order: outputs that cancel to near
    # zero (|y| <= 1e-2 against terms summing to ~1e2 in magnitude) differ by
    # more ulps than the rest, so they are held to the absolute bound only.
    theirs = F.linear(a, w, b)
    assert_bf16_close(to_np(out), to_np(theirs), max_ulp=1, frac_exact=0.98, atol=1e-2)


def test_adaln_table_without_silu():
    g = torch.Generator().manual_seed(3)
    temb = bf16_randn((4, 5120), g).cuda()
    w = bf16_randn((512, 5120), g, scale=0.02).cuda()
    out = kernels.adaln_table(temb, w, None, silu=False)
    assert np.array_equal(to_np(out), ref.adaln_table(to_np(temb), to_np(w)))


def test_adaln_table_rejects_unsupported():
    w = torch.zeros(64, 20, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="not supported"):
        kernels.adaln_table(torch.zeros(1, 20, device="cuda"), w)
    with pytest.raises(ValueError):
        kernels.adaln_table(torch.zeros(1, 24, device="cuda"), w)
