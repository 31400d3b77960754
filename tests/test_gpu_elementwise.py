"""GPU parity of the gated residual (bit-exact), SwiGLU (+quant) and
GELU-tanh (+quant) (bf16 tolerance) kernels (model/kernels.py:131-185)."""
import numpy as np
import pytest
import torch

import gpu_adapter as gpu
from helpers import assert_bf16_close, bf16_randn, to_np
from oracle import bf16, reference as ref

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("b,t,d,r", [(1, 512, 5120, 1), (2, 33, 5376, 6), (1, 7, 100, 2)])
def test_gated_residual_bit_exact(b, t, d, r):
    g = gen(b * t * d)
    x, u = bf16_randn((b, t, d), g), bf16_randn((b, t, d), g)
    table = bf16_randn((r, 6 * d), g, scale=0.1)
    idx = torch.randint(0, r, (t,), generator=g).numpy()
    for slot in (2, 5):
        got = gpu.gated_residual(to_np(x), to_np(u), to_np(table), idx, slot)
        assert np.array_equal(got, ref.gated_residual(to_np(x), to_np(u), to_np(table), idx, slot))


@pytest.mark.parametrize("rows,inner", [(64, 14336), (33, 160), (5, 100)])
def test_swiglu_within_tolerance(rows, inner):
    # Two bf16 roundings around the sigmoid: when the inner bf16(g*sigmoid(g))
    # lands one ulp apart, the outer product can move by two ulps (0.8%).
    p = bf16_randn((rows, 2 * inner), gen(rows + inner), scale=2.0)
    assert_bf16_close(gpu.swiglu(to_np(p)), ref.swiglu(to_np(p)), max_ulp=2, frac_exact=0.99,
                      atol=1e-4)


@pytest.mark.parametrize("rows,inner", [(64, 14336), (33, 160), (5, 100)])
def test_swiglu_quant(rows, inner):
    p = bf16_randn((rows, 2 * inner), gen(rows * inner), scale=2.0)
    q, s = gpu.swiglu_quant(to_np(p))
    # exact: the quantizer applied to the kernel's own activations
    act = gpu.swiglu(to_np(p))
    q2, s2 = ref.quantize_rows(act.reshape(rows, inner))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    # against the oracle's activations: +-1 where an activation differs by an ulp
    rq, rs = ref.swiglu_quant(to_np(p))
    assert np.abs(q.astype(np.int32) - rq).max() <= 2


def test_gelu_tanh_within_tolerance():
    x = torch.cat([torch.linspace(-12, 12, 40001), torch.randn(1 << 16) * 3]).bfloat16()
    assert_bf16_close(gpu.gelu_tanh(to_np(x)), ref.gelu_tanh(to_np(x)), frac_exact=0.99,
                      atol=1e-4)


def test_gelu_closed_forms():
    x = bf16.from_f32(np.array([0.0, -0.0, 30.0, -30.0, 1.0], np.float32))
    y = bf16.to_f32(gpu.gelu_tanh(x))
    assert y[0] == 0 and y[2] == 30 and abs(y[3]) < 1e-20
    assert abs(y[4] - 0.8411920071) < 4e-3


@pytest.mark.parametrize("rows,width", [(64, 20480), (33, 5120), (7, 20488), (3, 1000), (5, 100),
                                        (2, 41000)])
def test_gelu_quant_equals_gelu_then_quantize(rows, width):
    """One pass equals the two kernels it fuses bit for bit (vector path for
    widths divisible by 8 up to 16 chunks per thread, element-wise beyond),
    and stays within +-2 of the oracle's GELU then quantizer."""
    x = bf16_randn((rows, width), gen(rows * width + 1), scale=3.0, outliers=0.01)
    q, s = gpu.gelu_quant(to_np(x))
    act = gpu.gelu_tanh(to_np(x))
    q2, s2 = gpu.quantize_rows(act.reshape(rows, width))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    rq, rs = ref.quantize_rows(ref.gelu_tanh(to_np(x)).reshape(rows, width))
    assert np.abs(q.astype(np.int32) - rq).max() <= 2
    np.testing.assert_allclose(s, rs.reshape(-1), rtol=1e-2)


def test_gelu_quant_closed_forms():
    """A zero row quantizes to zeros with scale 1e-8/127; where GELU is the
    identity in bf16 (x >= 10) the row quantizes as x itself; where it
    underflows (x <= -30) the row is zero."""
    x = np.zeros((3, 64), np.float32)
    x[1] = np.linspace(10, 40, 64)
    x[2] = -np.linspace(30, 60, 64)
    xb = bf16.from_f32(x)
    q, s = gpu.gelu_quant(xb)
    assert not q[0].any() and s[0] == np.float32(np.float32(1e-8) / np.float32(127))
    q1, s1 = ref.quantize_rows(xb[1:2])
    assert np.array_equal(q[1], q1[0]) and s[1] == s1[0]
    assert not q[2].any()


@torch.inference_mode()
def test_gelu_quant_after_bf16_gemm_equals_gelu_epilogue():
    """The FFN-up GEMM with the bf16 epilogue followed by gelu_quant gives the
    same int8 rows and scales as the GEMM's GELU epilogue followed by the
    quantizer, at the C3 FFN width."""
    from lynnreal_omni_amd import int8_gemm, kernels
    g = gen(20)
    m, k, n = 384, 5120, 20480
    x = bf16_randn((m, k), g, outliers=0.01).cuda()
    q, s = kernels.quantize_rows(x)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).cuda()
    cs = (torch.rand(n, generator=g) * 4e-3 + 1e-3).cuda()
    b = (0.02 * torch.randn(n, generator=g)).bfloat16().cuda()
    fused_q, fused_s = kernels.quantize_rows(int8_gemm.int8_matmul(q, w.t(), s, cs, b, activation="gelu_tanh"))
    split_q, split_s = kernels._gelu_quant_int8(int8_gemm.int8_matmul(q, w.t(), s, cs, b))
    assert torch.equal(fused_q, split_q) and torch.equal(fused_s, split_s)
