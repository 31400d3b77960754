"""GPU parity of the split-K schedule of the INT8 GEMM (lr_int8_gemm_ws).

Split-K divides K over several workgroups per output tile, which write int32
partial sums to a workspace; a second kernel adds them and applies the
epilogue. Integer sums are exact in any order, so every split must equal the
oracle's int_mm (model/int8_gemm.py:13-46 restated) and the unsplit GEMM bit
for bit, including each epilogue (bf16 + bias, GELU-tanh, gated residual).
"""
import numpy as np
import pytest
import torch

from helpers import bf16_randn
from lynnreal_omni_amd import _lib, int8_gemm
from oracle import reference as ref
from oracle import torch_path as tp

pytestmark = pytest.mark.gpu

SPLIT_TILES = [(64, 80), (128, 160), (256, 80), (128, 128), (64, 128), (256, 256), (256, 192),
               (192, 256), "256x256_w4x2"]


def gen(seed):
    return torch.Generator().manual_seed(seed)


def rand_i8(shape, g):
    return torch.randint(-127, 128, shape, dtype=torch.int8, generator=g)


@pytest.mark.parametrize("tile", SPLIT_TILES, ids=str)
@pytest.mark.parametrize("m,n,k,splits", [
    (256, 5120, 1280, 2), (129, 520, 1024, 3), (300, 2056, 1280, 10), (64, 264, 640, 5),
    (1, 8, 256, 2), (700, 900, 2048, 7),
])
def test_split_int32_bit_exact(m, n, k, splits, tile):
    """Every tile in 2..10 slices (slices of unequal length where the k-step
    count does not divide), ragged M and N, against the oracle's int_mm."""
    g = gen(m + 3 * n + 7 * k + splits)
    a, w = rand_i8((m, k), g), rand_i8((n, k), g)
    got = int8_gemm.int8_matmul_int32(a.cuda(), w.cuda().t(), tile=tile, splits=splits)
    assert np.array_equal(got.cpu().numpy(), ref.int_mm(a.numpy(), w.numpy()))


def _epilogue_case(m, n, k, epi, g):
    x = bf16_randn((m, k), g, outliers=0.01)
    q, qs = tp.quantize(x)
    w = rand_i8((n, k), g)
    cs = torch.rand(n, generator=g) * 4e-3 + 1e-3
    b = (0.02 * torch.randn(n, generator=g)).bfloat16()
    kw = {}
    if epi == "gelu":
        kw = {"activation": "gelu_tanh"}
    elif epi == "gated":
        kw = {"residual": bf16_randn((1, m, n), g).cuda(),
              "table": (0.1 * torch.randn(3, 6 * n, generator=g)).bfloat16().cuda(),
              "indices": torch.randint(0, 3, (m,), generator=g).cuda(), "gate_slot": 2}
    return (q.cuda(), w.cuda().t(), qs.cuda(), cs.cuda(), b.cuda()), kw, (q, qs, w, cs, b)


@pytest.mark.parametrize("epi", ["bf16", "gelu", "gated"])
@pytest.mark.parametrize("m,n,k,tile,splits", [
    (256, 5120, 2048, (128, 160), 4),   # the vector reduce (N % 8 == 0)
    (129, 1028, 1024, (64, 80), 3),     # N % 8 != 0: one output per thread
    (40, 2056, 1280, (128, 128), 5),
])
def test_split_epilogues_equal_unsplit(m, n, k, tile, splits, epi):
    """The reduce kernel's dequant, GELU and gated-residual arithmetic equals
    the one-pass epilogue bit for bit; the bf16 epilogue also equals the
    oracle's dequant."""
    args, kw, cpu = _epilogue_case(m, n, k, epi, gen(m + n + k + len(epi)))
    whole = int8_gemm.int8_matmul(*args, tile=tile, splits=1, **kw)
    split = int8_gemm.int8_matmul(*args, tile=tile, splits=splits, **kw)
    assert torch.equal(whole, split)
    if epi == "bf16":
        q, qs, w, cs, b = cpu
        assert torch.equal(split.cpu(), tp.epilogue(tp.int_mm(q, w), qs, cs.reshape(1, -1), b))


@torch.inference_mode()
def test_auto_split_long_k_skinny_whole_output():
    """The automatic schedule splits K for a few hundred rows at long K
    (BASELINE config 5's M = 256 with the FFN-down shape, K = 20480, N = 5120):
    whole int32 and bf16 outputs against the oracle."""
    m, n, k = 256, 5120, 20480
    assert _lib.load().lr_int8_gemm_workspace_size(m, n, k, 0, _lib.TILE_AUTO) == 4 * m * n * 4
    g = gen(20261201 + 4)
    args, _, (q, qs, w, cs, b) = _epilogue_case(m, n, k, "bf16", g)
    acc = int8_gemm.int8_matmul_int32(args[0], args[1])
    want_acc = tp.int_mm(q, w)
    assert torch.equal(acc.cpu(), want_acc)
    y = int8_gemm.int8_matmul(*args)
    assert torch.equal(y.cpu(), tp.epilogue(want_acc, qs, cs.reshape(1, -1), b))


def test_split_repeats_identically():
    """The workspace is reused across calls: two calls with different shapes
    in a row, then the first again, each equal to the unsplit result."""
    g = gen(5)
    shapes = [(256, 5120, 2560), (64, 1024, 1280), (256, 5120, 2560)]
    for m, n, k in shapes:
        a, w = rand_i8((m, k), g).cuda(), rand_i8((n, k), g).cuda().t()
        want = int8_gemm.int8_matmul_int32(a, w, tile=(128, 160), splits=1)
        got = int8_gemm.int8_matmul_int32(a, w, tile=(128, 160), splits=4)
        assert torch.equal(got, want)


def test_split_invalid_requests():
    g = gen(9)
    a, w = rand_i8((64, 1024), g).cuda(), rand_i8((128, 1024), g).cuda().t()
    with pytest.raises(ValueError, match="splits"):
        int8_gemm.int8_matmul_int32(a, w, splits=9)          # K / 128 = 8 slices at most
    with pytest.raises(ValueError, match="persistent"):
        int8_gemm.int8_matmul_int32(a, w, tile="persistent", splits=2)
    a2, w2 = rand_i8((64, 1040), g).cuda(), rand_i8((128, 1040), g).cuda().t()
    with pytest.raises(ValueError, match="128"):
        int8_gemm.int8_matmul_int32(a2, w2, splits=2)        # K % 128 != 0
    a3, w3 = rand_i8((64, 1024), g).cuda(), rand_i8((130, 1024), g).cuda().t()
    with pytest.raises(ValueError, match="N % 4"):
        int8_gemm.int8_matmul_int32(a3, w3, splits=2)
