"""GPU parity of the per-row INT8 quantizer (model/int8.py:66-67) and the
stand-alone dequant epilogue (model/kernels.py:27-46): bit-exact vs the oracle."""
import numpy as np
import pytest
import torch

import golden_check
import gpu_adapter as gpu
from helpers import bf16_randn, to_np
from oracle import bf16, reference as ref

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("rows,width", [
    (2048, 5120),      # C1 activations
    (256, 20480),      # FFN-down input width
    (37, 5376),        # real-model width
    (5, 317),          # ragged width (element-wise path)
    (3, 1),
    (4, 40000),        # wider than the register-resident kernel
    (1, 8),
])
def test_quantize_rows_bit_exact(rows, width):
    x = bf16_randn((rows, width), gen(rows + width), outliers=0.01)
    x[0] = 0
    q, s = gpu.quantize_rows(to_np(x))
    rq, rs = ref.quantize_rows(to_np(x))
    assert np.array_equal(q, rq)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_quantize_rows_division_hard_cases():
    """Rows where rint(x * (1/s)) != rint(x / s) and exact .5 ties: the
    kernel's reciprocal fast path must fall back to the IEEE quotient."""
    from test_oracle import _division_mismatches
    cases = _division_mismatches(limit=512)
    rows = np.zeros((len(cases), 64), np.float32)
    for i, (m, x, _) in enumerate(cases):
        rows[i, 0] = m
        rows[i, 1:] = x          # many lanes of the same hard value
    ties = np.array([[127.0] + [k + 0.5 for k in range(-63, 63)] + [0.0]], np.float32)
    x = bf16.from_f32(np.concatenate([rows, np.resize(ties, (1, 128))[:, :64]]))
    q, s = gpu.quantize_rows(x)
    rq, rs = ref.quantize_rows(x)
    assert np.array_equal(q, rq) and np.array_equal(s, rs)


def test_quantize_rows_full_size_c2():
    x = bf16_randn((12288, 5120), gen(20261202), outliers=0.01)
    q, s = gpu.quantize_rows(to_np(x))
    rq, rs = ref.quantize_rows(to_np(x))
    assert np.array_equal(q, rq) and np.array_equal(s, rs)


def test_quantize_rows_empty():
    out = gpu.quantize_rows(np.zeros((0, 64), np.uint16))
    assert out[0].shape == (0, 64) and out[1].shape == (0,)


@pytest.mark.parametrize("m,n,bias", [(64, 512, True), (33, 70, False), (7, 5120, True)])
def test_int8_epilogue_bit_exact(m, n, bias):
    g = gen(m * n)
    acc = torch.randint(-(2**30), 2**30, (m, n), dtype=torch.int32, generator=g).numpy()
    rs = (torch.rand(m, generator=g) / 127).numpy()
    cs = (torch.rand(n, generator=g) * 4e-3 + 1e-3).numpy()
    b = to_np((torch.randn(n, generator=g) * 0.02).bfloat16()) if bias else None
    assert np.array_equal(gpu.dequant(acc, rs, cs, b), ref.dequant(acc, rs, cs, b))


def test_golden_fixtures_on_gpu():
    golden_check.check_all(gpu.module)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("rows,width", [(64, 5120), (7, 1000), (3, 20480)])
def test_quantize_rows_fp16_fp32_rows(dtype, rows, width):
    """fp16 and fp32 rows (the Triton quantizer loads any float row as fp32,
    model/kernels.py:12) against the torch restatement of model/int8.py:66-67
    on the same values; the first row holds exact half-integer quotients."""
    from lynnreal_omni_amd import kernels
    from oracle import torch_path as tp
    g = gen(rows * 31 + width)
    x = torch.randn(rows, width, generator=g) * 3
    x[:, ::97] *= 20
    x[0] = torch.arange(width) % 255 - 127.0
    x[0, 1::2] += 0.5
    x[0, 0] = 127.0
    x = x.to(dtype)
    q, s = kernels.quantize_rows(x.cuda())
    want_q, want_s = tp.quantize(x)
    assert torch.equal(q.cpu(), want_q) and torch.equal(s.cpu(), want_s)


def test_other_dtypes_are_recoverable_failures():
    """The bf16-only row kernels refuse other float types with the error that
    acceleration.optional_kernel_failure treats as recoverable, so the fused
    block guard falls back instead of failing (model/fusion.py:101-116)."""
    import types
    from lynnreal_omni_amd import acceleration, kernels
    x = torch.randn(1, 16, 64, device="cuda")
    norm = types.SimpleNamespace(weight=torch.ones(64, device="cuda", dtype=torch.bfloat16), eps=1e-6)
    table = torch.zeros(1, 6 * 64, device="cuda", dtype=torch.bfloat16)
    idx = torch.zeros(16, dtype=torch.int64, device="cuda")
    for call in (lambda: kernels._rms_adaln(x, norm, table, idx, 0, 1),
                 lambda: kernels._rms_adaln_quant_int8(x, norm, table, idx, 0, 1),
                 lambda: kernels._gated_residual(x, x.bfloat16(), table, idx, 2),
                 lambda: kernels.quantize_rows(torch.zeros(4, 8, dtype=torch.float64, device="cuda"))):
        with pytest.raises(RuntimeError, match="not supported") as err:
            call()
        assert acceleration.optional_kernel_failure(err.value)
