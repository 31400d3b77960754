"""The C-ABI library loads and exports every entry point of include/lynnreal_amd.h.

No compute is launched: only argument validation paths that return before
any HIP call, so these run on a machine without a GPU.
"""
import ctypes
import pathlib
import re
import subprocess

import pytest

from lynnreal_omni_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lynnreal_amd.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t|const char\*)\s+(lr_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        pytest.fail(f"{_lib.library_path()} is not built; run __graft_entry__.build()")
    return _lib.load()


def test_header_declares_the_path():
    names = declared()
    for expected in ("lr_quantize_rows", "lr_int8_gemm", "lr_int8_epilogue", "lr_rms_adaln",
                     "lr_rms_adaln_quant", "lr_residual_rms_quant", "lr_gated_residual",
                     "lr_swiglu", "lr_swiglu_quant", "lr_gelu_tanh", "lr_abi_version",
                     "lr_last_error", "lr_device_supported"):
        assert expected in names


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())],
                         capture_output=True, text=True, check=True).stdout
    return set(re.findall(r"\s[TW]\s+(lr_\w+)$", out, re.M))


def test_exported_symbols_are_exactly_the_declared_ones(lib):
    """The header is the whole ABI: nothing declared is missing from the
    library, and the library exports no lr_* entry point the header lacks
    (such as a tuning hook with process-global state)."""
    names = set(declared())
    got = exported()
    assert sorted(names - got) == [], "declared but not exported"
    assert sorted(got - names) == [], "exported but not declared"
    for name in names:
        assert hasattr(lib, name)


def test_python_prototypes_are_exactly_the_declared_ones():
    names = set(declared()) - {"lr_last_error", "lr_int8_gemm_workspace_size"}
    assert set(_lib.SIGNATURES) == names


def test_abi_version(lib):
    assert lib.lr_abi_version() == _lib.ABI_VERSION


def test_invalid_arguments_return_einval_without_a_gpu(lib):
    rc = lib.lr_quantize_rows(None, -1, 8, None, None, None)
    assert rc == _lib.LR_EINVAL
    assert b"negative shape" in lib.lr_last_error()
    rc = lib.lr_int8_gemm(None, None, 1, 1, 4, 4, 4, None, None, None, None, 99, None, None, 0, 0,
                          None, 0, 0, 0, None)
    assert rc == _lib.LR_EINVAL and b"epilogue" in lib.lr_last_error()
    rc = lib.lr_int8_gemm(None, None, 1, 1, 4, 4, 4, None, None, None, None, 0, None, None, 0, 0,
                          None, 0, 0, 0, None)
    assert rc == _lib.LR_EINVAL and b"null" in lib.lr_last_error()
    rc = lib.lr_rms_adaln(None, None, None, None, None, 4, 0, 8, 1, 48, 0, 1, 1e-6, None)
    assert rc == _lib.LR_EINVAL
    # table too narrow for slot 4 of hidden 8
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.lr_rms_adaln_quant(p, p, p, p, p, p, 4, 4, 8, 1, 32, 3, 4, 1e-6, None)
    assert rc == _lib.LR_EINVAL and b"too small" in lib.lr_last_error()
    # empty inputs are a no-op
    assert lib.lr_quantize_rows(None, 0, 8, None, None, None) == _lib.LR_OK


def test_status_mapping(lib):
    lib.lr_quantize_rows(None, -1, 8, None, None, None)
    with pytest.raises(ValueError, match="negative shape"):
        _lib.raise_for(_lib.LR_EINVAL, "lr_quantize_rows")
    with pytest.raises(RuntimeError, match="not supported"):
        _lib.raise_for(_lib.LR_EUNSUPPORTED, "x")
    import torch
    with pytest.raises(torch.cuda.OutOfMemoryError):
        _lib.raise_for(_lib.LR_ENOMEM, "x")
    with pytest.raises(RuntimeError):
        _lib.raise_for(_lib.LR_EHIP, "x")
    _lib.raise_for(_lib.LR_OK, "x")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("LYNNREAL_AMD_LIBRARY", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()


def test_split_k_workspace_sizes_and_checks_without_a_gpu(lib):
    """lr_int8_gemm_workspace_size: S x M x N int32 slices for a split-K
    schedule, 0 otherwise; lr_int8_gemm_ws refuses a forced split without
    room for its slices before any launch."""
    size = lib.lr_int8_gemm_workspace_size
    assert size(256, 5120, 5120, 1, _lib.TILE_AUTO) == 0
    assert size(256, 5120, 5120, 4, _lib.TILE_AUTO) == 4 * 256 * 5120 * 4
    assert size(256, 5120, 20480, 0, _lib.TILE_AUTO) == 4 * 256 * 5120 * 4  # auto: long K, M <= 256
    assert size(256, 5120, 5120, 0, _lib.TILE_AUTO) == 0
    assert size(12288, 5120, 20480, 0, _lib.TILE_AUTO) == 0
    assert size(256, 5120, 5136, 2, _lib.TILE_AUTO) == 0                     # K % 128 != 0
    p = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    rc = lib.lr_int8_gemm_ws(p, p, 1, 1024, 64, 128, 1024, p, p, None, p, 0, None, None, 0, 0, None, 0, 0,
                             None, 0, 2, _lib.TILE_AUTO, None)
    assert rc == _lib.LR_EINVAL and b"workspace" in lib.lr_last_error()
    rc = lib.lr_int8_gemm_ws(p, p, 1, 1024, 64, 128, 1024, p, p, None, p, 0, None, None, 0, 0, None, 0, 0,
                             None, 0, 65, _lib.TILE_AUTO, None)
    assert rc == _lib.LR_EINVAL and b"splits" in lib.lr_last_error()
