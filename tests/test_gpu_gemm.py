"""GPU parity of the INT8 MFMA GEMM (model/int8_gemm.py:13-46, :84-163).

int32 accumulators bit-exact vs the oracle's int_mm; bf16 epilogue bit-exact
vs the oracle's dequant (the reference asserts the same equality against its
torch path, script/precompile.py:55-64); GELU-tanh within the bf16 tolerance;
gated residual bit-exact vs the reference's _gated_residual composition.
"""
import hashlib

import numpy as np
import pytest
import torch

import golden_check
import gpu_adapter as gpu
from helpers import assert_bf16_close, bf16_randn, to_np
from lynnreal_omni_amd import int8_gemm
from oracle import reference as ref

pytestmark = pytest.mark.gpu

TILES = [None, (256, 256), "256x256_w4x2", (256, 192), (256, 80), (64, 80), (128, 160), (192, 256), (256, 128), (128, 256), (128, 128), (64, 128),
         "persistent",
         "generic"]


def gen(seed):
    return torch.Generator().manual_seed(seed)


def rand_i8(shape, g):
    return torch.randint(-127, 128, shape, dtype=torch.int8, generator=g).numpy()


@pytest.mark.parametrize("tile", TILES, ids=str)
@pytest.mark.parametrize("m,n,k", [
    (1, 64, 64), (7, 80, 48), (256, 256, 64), (300, 520, 272), (257, 255, 1024), (129, 384, 5120 + 16),
    # K of one and two 128-byte k-steps: the operand rings issue DMAs past the last k-step
    (200, 136, 128), (65, 520, 256),
])
def test_int32_accumulators_bit_exact(m, n, k, tile):
    g = gen(m * 7 + n * 3 + k)
    a, w = rand_i8((m, k), g), rand_i8((n, k), g)
    assert np.array_equal(gpu.int_mm(a, w, tile=tile), ref.int_mm(a, w))


def test_extreme_values_reach_int32_range():
    k = 20480
    a = np.full((64, k), -127, np.int8)
    w = np.full((128, k), -127, np.int8)
    w[1::2] = 127
    out = gpu.int_mm(a, w)
    assert (out[:, 0::2] == 127 * 127 * k).all() and (out[:, 1::2] == -127 * 127 * k).all()


def test_generic_paths_any_k_and_strides():
    g = gen(11)
    a, w = rand_i8((33, 100), g), rand_i8((70, 100), g)         # K % 16 != 0
    assert np.array_equal(gpu.int_mm(a, w), ref.int_mm(a, w))
    # B contiguous as [K, N] (strides (N, 1)): the generic kernel
    at, bt = torch.from_numpy(a).cuda(), torch.from_numpy(np.ascontiguousarray(w.T)).cuda()
    out = int8_gemm.int8_matmul_int32(at, bt)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), ref.int_mm(a, w))


@pytest.mark.parametrize("tile", [None, (128, 128), "generic"], ids=str)
@pytest.mark.parametrize("m,n,k,bias", [(45, 96, 256, True), (300, 1000, 640, False), (1, 8, 16, True)])
def test_bf16_epilogue_bit_exact(m, n, k, bias, tile):
    g = gen(m + n + k)
    a, w = rand_i8((m, k), g), rand_i8((n, k), g)
    rs = (torch.rand(m, generator=g) / 127).numpy()
    cs = (torch.rand(n, generator=g) * 4e-3 + 1e-3).numpy()
    b = to_np((torch.randn(n, generator=g) * 0.02).bfloat16()) if bias else None
    y = gpu.linear(a, rs, w, cs, b, tile=tile)
    assert np.array_equal(y, ref.linear(a, rs, w, cs, b))


def test_gelu_epilogue_within_tolerance():
    g = gen(12)
    m, n, k = 200, 640, 512
    a, w = rand_i8((m, k), g), rand_i8((n, k), g)
    rs = (torch.rand(m, generator=g) / 127).numpy()
    cs = (torch.rand(n, generator=g) * 4e-3 + 1e-3).numpy()
    b = to_np((torch.randn(n, generator=g) * 0.02).bfloat16())
    y = gpu.linear(a, rs, w, cs, b, activation="gelu_tanh")
    expect = ref.gelu_tanh(ref.linear(a, rs, w, cs, b))
    assert_bf16_close(y, expect, frac_exact=0.99, atol=1e-4)


@pytest.mark.parametrize("tile", [None, (256, 256), "generic"], ids=str)
def test_gated_residual_epilogue_bit_exact(tile):
    g = gen(13)
    batch, t, d, k = 2, 37, 320, 256
    m = batch * t
    a, w = rand_i8((m, k), g), rand_i8((d, k), g)
    rs = (torch.rand(m, generator=g) / 127).numpy()
    cs = (torch.rand(d, generator=g) * 4e-3 + 1e-3).numpy()
    x = bf16_randn((batch, t, d), g)
    table = bf16_randn((6, 6 * d), g, scale=0.1)
    idx = torch.randint(0, 6, (t,), generator=g)
    y = gpu.linear(a, rs, w, cs, None, tile=tile, residual=to_np(x), table=to_np(table),
                   indices=idx.numpy(), gate_slot=5)
    plain = ref.linear(a, rs, w, cs).reshape(batch, t, d)
    expect = ref.gated_residual(to_np(x), plain, to_np(table), idx.numpy(), 5)
    assert np.array_equal(y.reshape(batch, t, d), expect)


@pytest.mark.parametrize("shape", list(golden_check.load_kat()), ids=str)
def test_reference_install_check_shapes(shape):
    """The reference's install-time shapes (script/precompile.py:50-64), digests
    of the torch path's outputs committed in tests/golden/golden_kat.json."""
    from golden.make_golden import kat_inputs
    m, n, k = map(int, shape.split("x"))
    a, w, rs, cs = kat_inputs(m, n, k)
    want = golden_check.load_kat()[shape]
    acc = gpu.int_mm(a.numpy(), w.numpy())
    assert hashlib.sha256(acc.tobytes()).hexdigest() == want["acc_sha256"]
    y = gpu.linear(a.numpy(), rs.numpy().reshape(-1), w.numpy(), cs.numpy().reshape(-1))
    assert hashlib.sha256(y.tobytes()).hexdigest() == want["y_sha256"]


@pytest.mark.parametrize("m,n,k", [(16385, 21504, 5376), (16385, 5376, 7168),
                                   (49153, 28672, 5376), (16385, 5376, 14336)], ids=str)
def test_reference_full_m_install_shapes(m, n, k):
    """The full-M shapes of the reference's install check (script/precompile.py:
    51-53: the Flash model's QKV, out, FFN-up and FFN-down GEMMs with the
    16385-row and 49153-row tails) with the check it makes there (:55-64): the
    bf16 product equals the torch path's dequant of torch._int_mm, on the whole
    output. The int32 accumulators also pass the row- and column-sum closed
    forms, and sampled rows (both ends, so the one-row last tile) equal the C
    oracle."""
    from oracle import torch_path as tp
    g = torch.Generator(device="cuda").manual_seed(219)
    a = torch.randint(-127, 128, (m, k), device="cuda", dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (n, k), device="cuda", dtype=torch.int8, generator=g)
    rs = torch.rand(m, 1, device="cuda", generator=g) / 127
    cs = torch.rand(1, n, device="cuda", generator=g) / 127
    acc = int8_gemm.int8_matmul_int32(a, w.t())
    a64, w64 = a.to(torch.int64), w.to(torch.int64)
    assert torch.equal(acc.to(torch.int64).sum(dim=1), (a64 * w64.sum(dim=0)).sum(dim=1))
    assert torch.equal(acc.to(torch.int64).sum(dim=0), (w64 * a64.sum(dim=0)).sum(dim=1))
    del a64, w64
    assert torch.equal(acc, torch._int_mm(a, w.t()))
    y = int8_gemm.int8_matmul(a, w.t(), rs, cs)
    assert torch.equal(y, tp.epilogue(acc, rs, cs))
    rows = torch.cat([torch.arange(0, 24), torch.randint(24, m - 24, (16,)), torch.arange(m - 24, m)])
    a_rows = a[rows.cuda()].cpu().numpy()
    w_np = w.cpu().numpy()
    assert np.array_equal(acc[rows.cuda()].cpu().numpy(), ref.int_mm(a_rows, w_np))
    expect = ref.linear(a_rows, rs[rows.cuda()].cpu().numpy(), w_np, cs.cpu().numpy())
    assert np.array_equal(to_np(y[rows.cuda()]), expect)


def test_north_star_shape_whole_product():
    """M=12288, K=5120, N=20480: sampled rows equal the C oracle, every row
    sum and column sum equals its closed form by linearity, a second run gives
    the same output, and the whole int32 product equals torch._int_mm on the
    GPU (hipBLASLt's INT8 GEMM, an independent implementation whose results are
    exact integers); a difference from torch._int_mm is reported with the
    exact products at the first differing elements."""
    g = gen(14)
    m, n, k = 12288, 20480, 5120
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g).cuda()
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).cuda()
    acc = int8_gemm.int8_matmul_int32(a, w.t())
    rows = torch.cat([torch.arange(0, 64), torch.randint(64, m - 64, (64,), generator=g),
                      torch.arange(m - 64, m)])
    got = acc[rows.cuda()].cpu().numpy()
    expect = ref.int_mm(a[rows.cuda()].cpu().numpy(), w.cpu().numpy())
    assert np.array_equal(got, expect)
    a64, w64 = a.to(torch.int64), w.to(torch.int64)
    # sums by linearity: sum_n acc[m, n] = sum_k a[m, k] * (sum_n w[n, k]) and
    # sum_m acc[m, n] = sum_k (sum_m a[m, k]) * w[n, k]; a single wrong element
    # changes both its row's and its column's sum
    assert torch.equal(acc.to(torch.int64).sum(dim=1), (a64 * w64.sum(dim=0)).sum(dim=1))
    assert torch.equal(acc.to(torch.int64).sum(dim=0), (w64 * a64.sum(dim=0)).sum(dim=1))
    del a64, w64
    again = int8_gemm.int8_matmul_int32(a, w.t())
    assert torch.equal(acc, again), f"{int((acc != again).sum())} elements differ between two runs"
    del again
    other = torch._int_mm(a, w.t())
    bad = (acc != other).nonzero()
    if bad.numel():
        pos = bad[:16].cpu()
        exact = [int((a[r].to(torch.int64) * w[c].to(torch.int64)).sum()) for r, c in pos.tolist()]
        ours = acc[pos[:, 0].cuda(), pos[:, 1].cuda()].cpu().tolist()
        theirs = other[pos[:, 0].cuda(), pos[:, 1].cuda()].cpu().tolist()
        detail = (f"{bad.shape[0]} elements differ from torch._int_mm; first (row, col, ours, "
                  f"_int_mm, exact): {list(zip(pos.tolist(), ours, theirs, exact))}")
        assert ours == exact, "kernel wrong: " + detail
        assert theirs == exact, "torch._int_mm wrong: " + detail


@pytest.mark.parametrize("tile", [None, (256, 256), "256x256_w4x2"], ids=str)
def test_north_star_shape_repeats_identically(tile):
    """The same launch repeated ten times back to back on one stream gives the
    same bytes every time, int32 and bf16 + GELU (integer accumulation has one
    answer, so any difference is a race in the kernel's LDS or DMA schedule);
    the first run's int32 row sums equal their closed form."""
    g = torch.Generator(device="cuda").manual_seed(23)
    m, n, k = 12288, 20480, 5120
    a = torch.randint(-127, 128, (m, k), device="cuda", dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (n, k), device="cuda", dtype=torch.int8, generator=g)
    rs = torch.rand(m, device="cuda", generator=g) / 127 / 40
    cs = torch.rand(n, device="cuda", generator=g) / 127
    bias = (0.02 * torch.randn(n, device="cuda", generator=g)).bfloat16()
    first = int8_gemm.int8_matmul_int32(a, w.t(), tile=tile)
    expect_rows = (a.to(torch.int64) * w.to(torch.int64).sum(dim=0)).sum(dim=1)
    assert torch.equal(first.to(torch.int64).sum(dim=1), expect_rows)
    for rep in range(9):
        again = int8_gemm.int8_matmul_int32(a, w.t(), tile=tile)
        assert torch.equal(first, again), f"repeat {rep + 1}: {int((first != again).sum())} int32 differ"
    del again
    y0 = int8_gemm.int8_matmul(a, w.t(), rs, cs, bias, tile=tile, activation="gelu_tanh")
    for rep in range(9):
        y = int8_gemm.int8_matmul(a, w.t(), rs, cs, bias, tile=tile, activation="gelu_tanh")
        assert torch.equal(y0, y), f"repeat {rep + 1}: {int((y0 != y).sum())} bf16 differ"


@pytest.mark.parametrize("tile", TILES, ids=str)
def test_every_tile_repeats_identically(tile):
    """Every tile, C1's shape (M=2048, K=5120, N=5120): ten back-to-back
    launches give the same int32 and bf16 + GELU bytes, and the int32 result
    equals torch._int_mm."""
    g = torch.Generator(device="cuda").manual_seed(29)
    m, n, k = 2048, 5120, 5120
    a = torch.randint(-127, 128, (m, k), device="cuda", dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (n, k), device="cuda", dtype=torch.int8, generator=g)
    rs = torch.rand(m, device="cuda", generator=g) / 127 / 40
    cs = torch.rand(n, device="cuda", generator=g) / 127
    bias = (0.02 * torch.randn(n, device="cuda", generator=g)).bfloat16()
    first = int8_gemm.int8_matmul_int32(a, w.t(), tile=tile)
    assert torch.equal(first, torch._int_mm(a, w.t()))
    y0 = int8_gemm.int8_matmul(a, w.t(), rs, cs, bias, tile=tile, activation="gelu_tanh")
    for rep in range(9):
        assert torch.equal(first, int8_gemm.int8_matmul_int32(a, w.t(), tile=tile)), f"int32 repeat {rep + 1}"
        y = int8_gemm.int8_matmul(a, w.t(), rs, cs, bias, tile=tile, activation="gelu_tanh")
        assert torch.equal(y0, y), f"repeat {rep + 1}: {int((y0 != y).sum())} bf16 differ"


def test_torch_matmul_agrees_on_gpu():
    """_torch_matmul (torch._int_mm on the GPU) and the MFMA kernel agree
    bit for bit, as the reference's install check demands."""
    g = gen(15)
    m, n, k = 96, 320, 256
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g).cuda()
    b = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).cuda().t()
    rs = (torch.rand(m, 1, generator=g) / 127).cuda()
    cs = (torch.rand(1, n, generator=g) / 127).cuda()
    try:
        expect = int8_gemm._torch_matmul(a, b, rs, cs, None)
    except RuntimeError as error:
        pytest.skip(f"torch._int_mm unavailable on this GPU: {error}")
    assert torch.equal(int8_gemm.int8_matmul(a, b, rs, cs), expect)


def test_empty_and_invalid():
    a = torch.zeros(0, 64, dtype=torch.int8, device="cuda")
    b = torch.zeros(32, 64, dtype=torch.int8, device="cuda").t()
    out = int8_gemm.int8_matmul(a, b, torch.ones(0, device="cuda"), torch.ones(32, device="cuda"))
    assert out.shape == (0, 32)
    with pytest.raises(ValueError):
        int8_gemm.int8_matmul(torch.zeros(4, 64, dtype=torch.int8, device="cuda"), b,
                              torch.ones(4, device="cuda"), torch.ones(31, device="cuda"))


def test_c4_shapes_beyond_2gib():
    """Benchmark config 4 shapes (T=65536): FFN-up output bf16 [65536, 20480]
    (2.7 GB), its per-row quantization (K=20480) and the FFN-down GEMM
    (K=20480). Rows at the start, middle and end, whose byte offsets pass
    2^31, are checked against the oracle."""
    from lynnreal_omni_amd import kernels
    g = torch.Generator(device="cuda").manual_seed(15)
    m, d, f = 65536, 5120, 20480
    a = torch.randint(-127, 128, (m, d), dtype=torch.int8, device="cuda", generator=g)
    rs = torch.rand(m, device="cuda", generator=g) / 127 + 1e-4
    w_up = torch.randint(-127, 128, (f, d), dtype=torch.int8, device="cuda", generator=g)
    cs_up = torch.rand(f, device="cuda", generator=g) * 4e-3 + 1e-3
    w_dn = torch.randint(-127, 128, (d, f), dtype=torch.int8, device="cuda", generator=g)
    rows = torch.cat([torch.arange(0, 32), torch.arange(m // 2 - 16, m // 2 + 16), torch.arange(m - 64, m)])
    rows_d = rows.cuda()
    y = int8_gemm.int8_matmul(a, w_up.t(), rs, cs_up)
    assert y.shape == (m, f)
    a_s, w_up_h = a[rows_d].cpu().numpy(), w_up.cpu().numpy()
    want_y = ref.dequant(ref.int_mm(a_s, w_up_h), rs[rows_d].cpu().numpy(), cs_up.cpu().numpy())
    assert np.array_equal(to_np(y[rows_d]), want_y)
    q, s = kernels.quantize_rows(y)
    want_q, want_s = ref.quantize_rows(want_y)
    assert np.array_equal(q[rows_d].cpu().numpy(), want_q)
    assert np.array_equal(s[rows_d].reshape(-1).cpu().numpy(), want_s)
    del y
    acc = int8_gemm.int8_matmul_int32(q, w_dn.t())
    assert np.array_equal(acc[rows_d].cpu().numpy(), ref.int_mm(want_q, w_dn.cpu().numpy()))


@pytest.mark.parametrize("m,n,k", [(1024, 768, 1024), (16385, 5376, 7168), (20000, 2560, 384),
                                   (8200, 2056, 256), (8200, 2052, 384)])
def test_int8_tma_entry_matches_int8_matmul(m, n, k):
    """model/int8_tma.py:33-41's entry point (the persistent GEMM): same output
    as int8_matmul, and the reference's tile tuples map onto HIP tiles. The
    long-M shapes (the reference's M >= 16384 regime) give each of the 256
    workgroups 3-6 tiles, with M and N tails; 8200 x 2056 x 256 gives some
    workgroups a second tile two k-steps long (the shortest streamed loop),
    after a full tile or an edge tile, and checks the GELU epilogue too;
    N = 2052 (not a multiple of 8) runs the loop with the direct-store
    epilogue over several tiles per workgroup."""
    from lynnreal_omni_amd import int8_tma
    g = gen(16 + m)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g).cuda()
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).cuda()
    rs = (torch.rand(m, 1, generator=g) / 127).cuda()
    cs = (torch.rand(1, n, generator=g) * 4e-3 + 1e-3).cuda()
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16().cuda()
    y = int8_tma.matmul(a, w.t(), rs, cs, bias)
    assert torch.equal(y, int8_gemm.int8_matmul(a, w.t(), rs, cs, bias))
    assert torch.equal(int8_tma.matmul(a, w.t(), rs, cs, bias, tile=(128, 128, 128, 8, 3)), y)
    rows = np.unique(np.r_[0, 1, 255, 256, m // 2, m - 257, m - 256, m - 1])
    want = ref.dequant(ref.int_mm(a[rows].cpu().numpy(), w.cpu().numpy()), rs[rows].cpu().numpy(),
                       cs.cpu().numpy(), to_np(bias))
    assert np.array_equal(to_np(y[rows]), want)
    if k == 256:
        gelu = int8_gemm.int8_matmul(a, w.t(), rs, cs, bias, tile="persistent", activation="gelu_tanh")
        assert torch.equal(gelu, int8_gemm.int8_matmul(a, w.t(), rs, cs, bias, tile=(128, 128),
                                                       activation="gelu_tanh"))


@pytest.mark.parametrize("act", [None, "gelu_tanh", "swiglu"])
def test_chunked_rows_equal_unchunked(act):
    """Row independence, as the reference's sampling-safety check demands
    (comfyui/.../tools/verify_sampling_safety.py:58-78: chunked == unchunked
    for act in none/swiglu/gelu_tanh): the quantized projection of a row
    block equals the same rows of the whole-batch result, bit for bit."""
    from lynnreal_omni_amd import kernels
    g = gen(17)
    m, n, k = 777, 1024, 512
    x = bf16_randn((m, k), g, outliers=0.01).cuda()
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).cuda()
    cs = (torch.rand(n, generator=g) * 4e-3 + 1e-3).cuda()
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16().cuda()

    def project(rows):
        q, s = kernels.quantize_rows(rows)
        y = int8_gemm.int8_matmul(q, w.t(), s, cs, bias, activation="gelu_tanh" if act == "gelu_tanh" else None)
        return kernels._swiglu(y) if act == "swiglu" else y

    whole = project(x)
    parts = torch.cat([project(x[i:i + 100].contiguous()) for i in range(0, m, 100)])
    assert torch.equal(whole, parts)
