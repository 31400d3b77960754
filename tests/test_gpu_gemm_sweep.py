"""A seeded sweep of the INT8 GEMM over odd shapes, every tile and every
epilogue (model/int8_gemm.py:13-46; the epilogues of model/kernels.py:27-46,
:131-153): M and N that are not tile multiples, K a multiple of 16 but not of
the 128-byte k-step (the per-lane DMA path) and K a multiple of it (the
scalar-offset DMA path), with and without bias. int32, bf16 and gated-residual
outputs are compared bit for bit with the oracle, GELU-tanh within the bf16
tolerance. Each case is small; the point is the number of distinct tails."""
import numpy as np
import pytest
import torch

import gpu_adapter as gpu
from helpers import assert_bf16_close, bf16_randn, to_np
from oracle import reference as ref

pytestmark = pytest.mark.gpu

TILES = [None, (256, 256), "256x256_w4x2", (256, 192), (256, 80), (64, 80), (128, 160), (192, 256), (256, 128), (128, 256), (128, 128), (64, 128),
         "persistent",
         "generic"]
EPILOGUES = ["int32", "bf16", "gelu_tanh", "gated"]


def _cases(count=4 * len(TILES), seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        m = int(rng.integers(1, 700))
        n = int(rng.integers(1, 90)) * 8            # the staged epilogue needs N % 8 == 0 ...
        if i % 4 == 3:
            n += 4                                  # ... and N % 8 == 4 takes the direct stores
        k = int(rng.integers(1, 80)) * 16
        # with T = len(TILES) = 14 tiles, tile t meets epilogues t, t + 3, t + 2 and
        # t + 1 (mod 4) in cases t, t + T, t + 2T and t + 3T: every tile meets every
        # epilogue once
        out.append((m, n, k, TILES[i % len(TILES)], EPILOGUES[(i + i // len(TILES)) % len(EPILOGUES)],
                    i % 3 != 0))
    return out


def _aligned_cases(seed=20261206):
    """K a multiple of 128 with M and N tails: one case per tile, every epilogue."""
    rng = np.random.default_rng(seed)
    out = []
    for i, tile in enumerate(TILES):
        m = int(rng.integers(1, 700))
        n = int(rng.integers(1, 90)) * 8 + (4 if i % 3 == 2 else 0)
        k = int(rng.integers(1, 12)) * 128
        out.append((m, n, k, tile, EPILOGUES[i % len(EPILOGUES)], i % 2 == 0))
    return out


@pytest.mark.parametrize("m,n,k,tile,epilogue,bias", _cases() + _aligned_cases(),
                         ids=lambda v: str(v) if not isinstance(v, tuple) else "x".join(map(str, v)))
def test_random_shape(m, n, k, tile, epilogue, bias):
    g = torch.Generator().manual_seed(m * 1000003 + n * 101 + k)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g).numpy()
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).numpy()
    if epilogue == "int32":
        assert np.array_equal(gpu.int_mm(a, w, tile=tile), ref.int_mm(a, w))
        return
    rs = (torch.rand(m, generator=g) / 127).numpy()
    cs = (torch.rand(n, generator=g) * 4e-3 + 1e-3).numpy()
    b = to_np((torch.randn(n, generator=g) * 0.02).bfloat16()) if bias else None
    if epilogue == "bf16":
        assert np.array_equal(gpu.linear(a, rs, w, cs, b, tile=tile), ref.linear(a, rs, w, cs, b))
    elif epilogue == "gelu_tanh":
        y = gpu.linear(a, rs, w, cs, b, tile=tile, activation="gelu_tanh")
        assert_bf16_close(y, ref.gelu_tanh(ref.linear(a, rs, w, cs, b)), frac_exact=0.99, atol=1e-4)
    else:
        rows = 3
        x = bf16_randn((1, m, n), g)
        table = bf16_randn((rows, 6 * n), g, scale=0.1)
        idx = torch.randint(0, rows, (m,), generator=g)
        y = gpu.linear(a, rs, w, cs, b, tile=tile, residual=to_np(x), table=to_np(table),
                       indices=idx.numpy(), gate_slot=2)
        plain = ref.linear(a, rs, w, cs, b).reshape(1, m, n)
        want = ref.gated_residual(to_np(x), plain, to_np(table), idx.numpy(), 2)
        assert np.array_equal(y.reshape(1, m, n), want)
