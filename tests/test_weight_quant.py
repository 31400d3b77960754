"""int8.quantize_weight, the float -> INT8 weight conversion of Int8Linear
(reference model/int8.py:9-11), pinned without restating its formula:

* on bf16 weights it must equal the C oracle's per-row quantizer applied to
  the weight rows (the same arithmetic: fp32 absmax / 127 by IEEE division,
  fp32 quotient rounded half to even, clamp to +-127), over random rows with
  outliers;
* hand-built rows whose scale is a power of two, so every quotient is exact
  and the expected integers are known: half-way values round to even,
  the absmax element maps to +-127, signs are symmetric;
* an all-zero row keeps scale 1e-8 / 127 and quantizes to zeros;
* an fp32 row where the fp32 quotient and the exact real quotient round to
  different integers, which a float64 division or a multiply by the
  reciprocal would get wrong.
"""
import numpy as np
import torch

from helpers import bf16_randn, to_np
from lynnreal_omni_amd.int8 import quantize_weight
from oracle import reference as ref


def test_bf16_weights_match_the_oracle_row_quantizer():
    g = torch.Generator().manual_seed(31)
    w = bf16_randn((300, 1024), g, scale=0.02, outliers=0.01)
    q, s = quantize_weight(w)
    rq, rs = ref.quantize_rows(to_np(w))
    assert q.dtype == torch.int8 and s.dtype == torch.float32 and s.shape == (300, 1)
    assert np.array_equal(q.numpy(), rq)
    assert np.array_equal(s.reshape(-1).numpy(), rs)


def test_power_of_two_scales_round_half_to_even():
    # absmax 127 * 2^-7 -> scale exactly 2^-7; entries k/2 * 2^-7 are exact ties.
    unit = 2.0 ** -7
    halves = [0.5, 1.5, 2.5, 3.5, 126.5, -0.5, -1.5, -2.5, -126.5, 127.0, -127.0, 0.0, 3.0]
    expect = [0, 2, 2, 4, 126, 0, -2, -2, -126, 127, -127, 0, 3]
    row = torch.tensor([h * unit for h in halves], dtype=torch.float32)
    for sign in (1.0, -1.0):
        q, s = quantize_weight((sign * row).reshape(1, -1))
        assert float(s) == unit
        assert q.reshape(-1).tolist() == [int(sign * e) if e else 0 for e in expect]


def test_zero_row_and_symmetry():
    w = torch.zeros(2, 16)
    w[1, 3] = -5.0
    q, s = quantize_weight(w)
    assert float(s[0]) == np.float32(np.float32(1e-8) / np.float32(127))
    assert (q[0] == 0).all()
    assert q[1, 3] == -127 and (q[1].abs().sum() == 127)
    g = torch.Generator().manual_seed(32)
    w = torch.randn(64, 256, generator=g)
    qp, sp = quantize_weight(w)
    qn, sn = quantize_weight(-w)
    assert torch.equal(sp, sn) and torch.equal(qn, -qp)


def test_fp32_quotient_is_rounded_before_rint():
    """Among fp32 values x of one row with absmax a, find those whose real
    quotient x / (a / 127) is not a tie but whose fp32 rounding is exactly
    k + 1/2, and where round-half-even of that tie differs from rounding the
    real quotient: the conversion must follow the fp32 quotient."""
    a = np.float32(0.7)
    scale = np.float32(a / np.float32(127))
    # fp32 values within 64 ulps of every tie point (k + 1/2) * scale, k = 0..125
    ties = ((np.arange(126) + 0.5) * np.float64(scale)).astype(np.float32).view(np.int32)
    x = (ties[:, None] + np.arange(-64, 65, dtype=np.int32)[None, :]).reshape(-1).view(np.float32)
    quo32 = (x / scale).astype(np.float32)
    quo64 = x.astype(np.float64) / np.float64(scale)
    tie = (quo32 % 1) == 0.5
    even = 2 * np.round(quo32.astype(np.float64) / 2)      # half-even of an exact tie
    nearest = np.floor(quo64 + 0.5)                          # rounding the real quotient
    pick = np.flatnonzero(tie & ((quo64 % 1) != 0.5) & (even != nearest))[:8]
    assert pick.size, "no value where the fp32 quotient decides the rounding"
    row = torch.from_numpy(np.concatenate([[a], x[pick]]).astype(np.float32)).reshape(1, -1)
    q, s = quantize_weight(row)
    assert float(s) == float(scale)
    assert q[0, 1:].tolist() == even[pick].astype(int).tolist()
    assert q[0, 1:].tolist() != nearest[pick].astype(int).tolist()
