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


def test_fast_call_shim_is_built_and_bound():
    """build() puts the CPython fast-call module beside the library; the
    integer-argument entry points go through it and the ones with float
    arguments (eps) stay on ctypes."""
    from lynnreal_omni_amd import _pycall  # noqa: F401  (fails loudly if not built)
    assert _lib._pycall is not None
    fast = _lib._bind("lr_int8_gemm_ws")
    slow = _lib._bind("lr_rms_adaln")
    assert not isinstance(fast, ctypes._CFuncPtr) and isinstance(slow, ctypes._CFuncPtr)


def test_fast_call_matches_ctypes_statuses(lib):
    """The same invalid calls give the same statuses and messages through the
    shim as through ctypes (validation runs before any GPU call)."""
    cases = [
        ("lr_quantize_rows", (None, -1, 8, None, None, None), b"negative shape"),
        ("lr_quantize_rows", (None, 1, 8, None, None, None), b"null"),
        ("lr_int8_gemm", (None, None, 1, 1, 4, 4, 4, None, None, None, None, 99, None, None, 0, 0,
                          None, 0, 0, 0, None), b"epilogue"),
        ("lr_int8_gemm_ws", (None, None, 1, 1, 4, 4, 4, None, None, None, None, 0, None, None, 0, 0,
                             None, 0, 0, None, 0, 0, 99, None), b"unknown tile"),
        ("lr_int8_gemm_ws", (None, None, 1, 1, 4, 4, 4, None, None, None, None, 0, None, None, 0, 0,
                             None, 0, 0, None, -5, 0, 0, None), b"workspace"),
        ("lr_gelu_quant", (None, None, None, 3, 0, None), b"bad shape"),
    ]
    for name, args, message in cases:
        fast = _lib._bind(name)(*args)
        fast_msg = lib.lr_last_error()
        slow = getattr(lib, name)(*args)
        assert fast == slow == _lib.LR_EINVAL and message in fast_msg and fast_msg == lib.lr_last_error()
    assert _lib._bind("lr_quantize_rows")(None, 0, 8, None, None, None) == _lib.LR_OK


def test_fast_call_passes_every_argument(tmp_path):
    """All 24 argument slots of the shim, mixing int and int64_t parameters as
    the GEMM entry point does, with negative values, None (0) and large
    pointer-like values, reach a C function intact (a helper compiled here)."""
    import shutil
    from lynnreal_omni_amd import _pycall
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "probe.c"
    params = ", ".join(f"{'int' if i % 3 == 1 else 'long long'} a{i}" for i in range(24))
    body = " ".join(f"h = h * 1000003ULL ^ (unsigned long long)(long long)a{i};" for i in range(24))
    src.write_text("static unsigned long long h;\n"
                   f"int probe({params}) {{ h = 0; {body} return (int)(h ^ (h >> 32)); }}\n")
    so = tmp_path / "libprobe.so"
    subprocess.run([cc, "-O1", "-shared", "-fPIC", str(src), "-o", str(so)], check=True)
    fn = ctypes.CDLL(str(so)).probe
    address = ctypes.cast(fn, ctypes.c_void_p).value
    values = [(-1) ** i * (i * 7919 + 3) for i in range(24)]
    values[2], values[5], values[8] = None, 0x7fff_dead_beef_0000, -(2 ** 40)
    values[10] = 2 ** 31 - 1   # an int parameter at its maximum
    expect_h = 0
    for i, v in enumerate(values):
        x = 0 if v is None else v
        if i % 3 == 1:
            x = ((x + 2 ** 31) % 2 ** 32) - 2 ** 31   # what an int parameter reads
        expect_h = ((expect_h * 1000003) % 2 ** 64) ^ (x % 2 ** 64)
    folded = (expect_h ^ (expect_h >> 32)) % 2 ** 32
    expect = folded - 2 ** 32 if folded >= 2 ** 31 else folded
    assert _pycall.call(address, *values) == expect
    with pytest.raises(TypeError):
        _pycall.call(address, 1.5)
    with pytest.raises(TypeError):
        _pycall.call(address, *range(25))
