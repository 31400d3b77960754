"""GPU parity of the fused Q/K RMSNorm + RoPE kernel (model/kernels.py:187-257,
345-402; launched at model/fusion.py:35-52): bit-exact vs the oracle, which
uses the kernel's defined sum order, on strided Q/K views of a fused QKV
tensor (the reference's install check, script/precompile.py:12-33, uses
such views with a non-aligned token count); and close to the reference's
Triton semantics (torch reduction, rsqrt), to the bound that a 1-ulp change
of the normalized value propagates to through the rotation."""
import numpy as np
import pytest
import torch

from helpers import assert_rope_close, bf16_randn, to_np
from lynnreal_omni_amd import kernels
from oracle import bf16, reference as ref, torch_path as tp

pytestmark = pytest.mark.gpu

CASES = [
    # batch, tokens, heads (q and k each), head_dim, rotary_dim
    (1, 128, 4, 128, 16),    # precompile KAT shapes
    (2, 137, 4, 128, 16),
    (2, 137, 4, 128, 128),   # full-width paired RoPE
    (1, 77, 40, 128, 64),
    (1, 300, 8, 64, 64),
    (2, 31, 5, 64, 32),
    (1, 50, 6, 32, 16),
    (1, 19, 3, 128, 0),      # RMSNorm only
    (1, 33, 5, 128, 48),     # pair distances that are not powers of two: DPP row shifts
    (2, 21, 3, 128, 80),
    (1, 40, 4, 128, 96),
    (1, 17, 6, 128, 112),
    (1, 29, 7, 64, 48),
]


@pytest.mark.parametrize("batch,tokens,heads,dim,rot", CASES)
def test_qk_norm_rope_bit_exact(batch, tokens, heads, dim, rot):
    g = torch.Generator().manual_seed(batch * 1000 + tokens + dim + rot)
    qkv = bf16_randn((batch, tokens, 3 * heads, dim), g, outliers=0.01)
    qw = (1 + 0.1 * torch.randn(dim, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(dim, generator=g)).bfloat16()
    phase = torch.randn(tokens, rot, generator=g) * 3
    cos, sin = phase.cos(), phase.sin()
    dev = qkv.cuda()
    q, k = dev[:, :, :heads], dev[:, :, heads:2 * heads]          # strided views
    qo, ko = kernels.qk_norm_rope(q, k, qw.cuda(), kw.cuda(), (cos.cuda(), sin.cuda()), 1e-6)
    torch.cuda.synchronize()
    assert qo.is_contiguous() and qo.shape == q.shape
    want_q, want_k = ref.qk_norm_rope(to_np(qkv[:, :, :heads]), to_np(qkv[:, :, heads:2 * heads]),
                                      to_np(qw), to_np(kw), cos.numpy(), sin.numpy(), 1e-6)
    assert np.array_equal(to_np(qo.cpu()), want_q)
    assert np.array_equal(to_np(ko.cpu()), want_k)
    # and the reference's own semantics (torch reduction order, rsqrt)
    tq, tk = tp.qk_norm_rope(qkv[:, :, :heads], qkv[:, :, heads:2 * heads], qw, kw, cos, sin, 1e-6)
    for o, t in ((qo, tq), (ko, tk)):
        assert_rope_close(to_np(o.cpu()), to_np(t), rot)


def test_qk_norm_rope_contiguous_inputs_and_bf16_tables():
    g = torch.Generator().manual_seed(7)
    q = bf16_randn((1, 64, 8, 128), g)
    k = bf16_randn((1, 64, 8, 128), g)
    w = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    phase = torch.randn(64, 128, generator=g)
    cos, sin = phase.cos().bfloat16(), phase.sin().bfloat16()     # bf16 tables widen exactly
    qo, ko = kernels.qk_norm_rope(q.cuda(), k.cuda(), w.cuda(), w.cuda(), (cos.cuda(), sin.cuda()), 1e-5)
    want_q, want_k = ref.qk_norm_rope(to_np(q), to_np(k), to_np(w), to_np(w), cos.float().numpy(),
                                      sin.float().numpy(), 1e-5)
    assert np.array_equal(to_np(qo.cpu()), want_q) and np.array_equal(to_np(ko.cpu()), want_k)


def test_qk_norm_rope_rejects_bad_arguments():
    q = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16, device="cuda")
    w = torch.ones(128, dtype=torch.bfloat16, device="cuda")
    odd = torch.zeros(4, 15, device="cuda")
    with pytest.raises(ValueError):
        kernels.qk_norm_rope(q, q, w, w, (odd, odd), 1e-6)
    big = torch.zeros(4, 256, device="cuda")
    with pytest.raises(ValueError):
        kernels.qk_norm_rope(q, q, w, w, (big, big), 1e-6)
    r24 = torch.zeros(4, 24, device="cuda")          # not a multiple of 16
    with pytest.raises(RuntimeError, match="not supported"):
        kernels.qk_norm_rope(q, q, w, w, (r24, r24), 1e-6)
    q96 = torch.zeros(1, 4, 2, 96, dtype=torch.bfloat16, device="cuda")
    w96 = torch.ones(96, dtype=torch.bfloat16, device="cuda")
    r48 = torch.zeros(4, 48, device="cuda")          # head_dim 96: not a supported width
    with pytest.raises(RuntimeError, match="not supported"):
        kernels.qk_norm_rope(q96, q96, w96, w96, (r48, r48), 1e-6)
