"""lr_int8_gemm_noalloc: the split-K GEMM with its slices in the library's
own device array, for callers that cannot allocate.

Called through the C ABI and checked against lr_int8_gemm_ws (the entry point
that takes a workspace) bit for bit, on two calls in a row whose second input
is smaller, then refused beyond the array's size.
"""
import pytest
import torch

from lynnreal_omni_amd import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _inputs(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g).cuda()
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g).cuda()
    rs = (torch.rand(m, generator=g) * 0.05 + 0.01).cuda()
    cs = (torch.rand(n, generator=g) * 4e-3 + 1e-3).cuda()
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16().cuda()
    return a, w, rs, cs, bias


def _args(a, w, rs, cs, bias, out, epilogue):
    m, k = a.shape
    n = w.shape[0]
    raw = epilogue == _lib.EPI_RAW_INT32
    return (a.data_ptr(), w.data_ptr(), 1, k, m, n, k, None if raw else rs.data_ptr(),
            None if raw else cs.data_ptr(), None if raw else bias.data_ptr(), out.data_ptr(), epilogue,
            None, None, 0, 0, None, 0, 0)


@pytest.mark.parametrize("epilogue", [_lib.EPI_BF16, _lib.EPI_RAW_INT32])
def test_noalloc_equals_workspace_entry_point(epilogue):
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    dtype = torch.int32 if epilogue == _lib.EPI_RAW_INT32 else torch.bfloat16
    # The automatic schedule splits K for both shapes (a few hundred rows at
    # long K); the second call's slices are smaller than the first's.
    for m, n, k in ((256, 5120, 20480), (128, 2048, 16384)):
        need = lib.lr_int8_gemm_workspace_size(m, n, k, 0, _lib.TILE_AUTO)
        assert 0 < need <= SCRATCH_BYTES
        a, w, rs, cs, bias = _inputs(m, n, k, m + n + k)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        want = torch.empty(m, n, dtype=dtype, device="cuda")
        got = torch.full((m, n), 7, dtype=dtype, device="cuda")
        rc = lib.lr_int8_gemm_ws(*_args(a, w, rs, cs, bias, want, epilogue), ws.data_ptr(), need, 0,
                                 _lib.TILE_AUTO, stream)
        assert rc == _lib.LR_OK, lib.lr_last_error()
        rc = lib.lr_int8_gemm_noalloc(*_args(a, w, rs, cs, bias, got, epilogue), 0, _lib.TILE_AUTO, stream)
        assert rc == _lib.LR_OK, lib.lr_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_noalloc_forced_split_and_limit():
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    m, n, k = 300, 1000, 2048
    a, w, rs, cs, bias = _inputs(m, n, k, 3)
    want = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    got = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    need = lib.lr_int8_gemm_workspace_size(m, n, k, 5, _lib.TILE_AUTO)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    assert lib.lr_int8_gemm_ws(*_args(a, w, rs, cs, bias, want, _lib.EPI_BF16), ws.data_ptr(), need, 5,
                               _lib.TILE_AUTO, stream) == _lib.LR_OK
    assert lib.lr_int8_gemm_noalloc(*_args(a, w, rs, cs, bias, got, _lib.EPI_BF16), 5, _lib.TILE_AUTO,
                                    stream) == _lib.LR_OK
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # 16 slices of 300 x 2000 int32 need 38.4 MB, beyond the 32 MiB array:
    # refused before any launch, and the output is left alone.
    m, n, k = 300, 2000, 2048
    a, w, rs, cs, bias = _inputs(m, n, k, 4)
    out = torch.zeros(m, n, dtype=torch.bfloat16, device="cuda")
    assert lib.lr_int8_gemm_workspace_size(m, n, k, 16, _lib.TILE_AUTO) > SCRATCH_BYTES
    rc = lib.lr_int8_gemm_noalloc(*_args(a, w, rs, cs, bias, out, _lib.EPI_BF16), 16, _lib.TILE_AUTO, stream)
    assert rc == _lib.LR_EINVAL and b"maximum" in lib.lr_last_error()
    torch.cuda.synchronize()
    assert not out.any()
