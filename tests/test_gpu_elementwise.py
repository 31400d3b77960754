"""GPU parity of the gated residual (bit-exact), SwiGLU (+quant) and
GELU-tanh (bf16 tolerance) kernels (model/kernels.py:131-185)."""
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
