"""Conversions and comparison helpers shared by the tests."""
from __future__ import annotations

import numpy as np
import torch

from oracle import bf16


def to_np(t: torch.Tensor) -> np.ndarray:
    """Tensor -> numpy (bf16 as uint16 bit patterns)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def from_np(a: np.ndarray, device="cpu", dtype=None) -> torch.Tensor:
    """numpy -> tensor (uint16 arrays become bf16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    else:
        t = torch.from_numpy(a.copy())
    if dtype is not None:
        t = t.to(dtype)
    return t.to(device)


def bf16_randn(shape, gen, scale=1.0, outliers=0.0, outlier_scale=20.0):
    """bf16 N(0, scale^2) with a fraction of channels (last dim) multiplied."""
    x = torch.randn(*shape, generator=gen) * scale
    if outliers:
        width = shape[-1]
        count = max(1, int(round(width * outliers)))
        idx = torch.randperm(width, generator=gen)[:count]
        x[..., idx] *= outlier_scale
    return x.bfloat16()


def assert_bf16_close(actual_u16, expected_u16, *, max_ulp=1, frac_exact=0.999, rel=1e-2,
                      cos=0.9999, atol=0.0):
    """The bf16 tolerance: every element within `max_ulp` bf16 ulps (elements
    whose expected and actual magnitudes are both <= atol are exempt), at least
    `frac_exact` identical, max relative error <= rel (on |x| > 1e-3 of the
    max) and cosine similarity >= cos."""
    a = np.asarray(actual_u16, np.uint16).reshape(-1)
    e = np.asarray(expected_u16, np.uint16).reshape(-1)
    assert a.shape == e.shape
    ulp = bf16.ulp_distance(a, e)
    if atol:
        tiny = (np.abs(bf16.to_f32(a)) <= atol) & (np.abs(bf16.to_f32(e)) <= atol)
        ulp = np.where(tiny, 0, ulp)
    assert ulp.max() <= max_ulp, f"max ulp distance {ulp.max()}"
    exact = float((ulp == 0).mean())
    assert exact >= frac_exact, f"only {exact:.5f} identical"
    af, ef = bf16.to_f32(a).astype(np.float64), bf16.to_f32(e).astype(np.float64)
    big = np.abs(ef) > 1e-3 * np.abs(ef).max()
    if big.any():
        relerr = np.abs(af[big] - ef[big]) / np.abs(ef[big])
        assert relerr.max() <= rel, f"max rel err {relerr.max()}"
    denom = np.linalg.norm(af) * np.linalg.norm(ef)
    if denom > 0:
        assert float(af @ ef) / denom >= cos


def assert_rope_close(actual_u16, expected_u16, rotary_dim, frac_exact=0.99):
    """Tolerance for QK-RMSNorm + RoPE outputs whose sum of squares is
    reduced in a different order from the expected values.

    The normalized value n = bf16(x * rstd * w) may differ by one bf16 ulp.
    Unrotated dimensions are exactly n, so they stay within 1 ulp. A rotated
    output is bf16(a -/+ b) with a = bf16(n * c), b = bf16(n' * s), |c|, |s|
    <= 1: a 1-ulp change of n moves a (and b) by at most 2 ulps of their own
    magnitude, 2 * 2^-7 * |a|, and the output rounding adds 2^-8 * |out|. With
    |a|, |b| <= max |n| over the row, and rotation keeping each (n, n') pair's
    length, max |n| is within rounding of the largest output of the row:
      |out - expected| <= 2^-5 * max_row |expected| * 1.02 + 2^-7 * |expected|.
    Cancellation (a ~ b) makes a ulp count of the output meaningless there,
    hence the absolute bound. At least `frac_exact` must be identical."""
    a = np.asarray(actual_u16, np.uint16)
    e = np.asarray(expected_u16, np.uint16)
    assert a.shape == e.shape
    ulp = bf16.ulp_distance(a, e)
    assert float((ulp == 0).mean()) >= frac_exact, f"only {(ulp == 0).mean():.5f} identical"
    assert ulp[..., rotary_dim:].max(initial=0) <= 1, "unrotated dimensions beyond 1 ulp"
    if rotary_dim:
        af = bf16.to_f32(a[..., :rotary_dim]).astype(np.float64)
        ef = bf16.to_f32(e[..., :rotary_dim]).astype(np.float64)
        bound = 2.0 ** -5 * 1.02 * np.abs(ef).max(axis=-1, keepdims=True) + 2.0 ** -7 * np.abs(ef)
        worst = (np.abs(af - ef) - bound).max()
        assert worst <= 0, f"rotated output beyond the propagated bound by {worst}"
