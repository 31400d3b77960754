"""Capability probe and recoverable-error policy (drop-in for the relevant
parts of the reference's model/acceleration.py).

fastest_available() checks the gfx950 library on the current device with two
exact probes modelled on the reference's install-time checks
(script/precompile.py:50-77, model/acceleration.py:31-39): the MFMA GEMM
against the torch path, and residual_rms_quant against _gated_residual
followed by _rms_adaln_quant_int8.
"""
from __future__ import annotations

import types

import torch

_RECOVERABLE = ("not supported", "not implemented", "no kernel image", "invalid device function")


def optional_kernel_failure(error) -> bool:
    """True for compile/device-support failures a caller may fall back from;
    never for out-of-memory (model/acceleration.py:49-56)."""
    if isinstance(error, torch.cuda.OutOfMemoryError):
        return False
    origin = type(error).__module__
    if origin.startswith(("triton", "torch._dynamo", "torch._inductor")):
        return True
    text = str(error).lower()
    return any(marker in text for marker in _RECOVERABLE)


def _probe_gemm(device) -> bool:
    from .int8_gemm import _torch_matmul, int8_matmul
    gen = torch.Generator(device="cpu").manual_seed(219)
    m, n, k = 96, 320, 256
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=gen).to(device)
    b = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=gen).to(device).t()
    rs = (torch.rand(m, 1, generator=gen) / 127).to(device)
    cs = (torch.rand(1, n, generator=gen) / 127).to(device)
    return torch.equal(int8_matmul(a, b, rs, cs), _torch_matmul(a, b, rs, cs, None))


def _probe_residual(device) -> bool:
    from .kernels import _gated_residual, _rms_adaln_quant_int8, residual_rms_quant
    gen = torch.Generator(device="cpu").manual_seed(220)
    hidden = 192
    x = torch.randn(1, 32, hidden, generator=gen).bfloat16().to(device)
    update = torch.randn(1, 32, hidden, generator=gen).bfloat16().to(device)
    table = torch.randn(2, 6 * hidden, generator=gen).bfloat16().to(device)
    indices = (torch.arange(32) % 2).to(device)
    norm = types.SimpleNamespace(weight=torch.ones(hidden, dtype=torch.bfloat16, device=device), eps=1e-5)
    residual = _gated_residual(x, update, table, indices, 2)
    expected = (residual, *_rms_adaln_quant_int8(residual, norm, table, indices, 3, 4))
    actual = residual_rms_quant(x, update, norm, table, indices)
    return all(torch.equal(a, b) for a, b in zip(actual, expected))


def fastest_available(attention_backend=None):
    """Probe the fused W8A8 kernels on the current GPU.

    Returns {"fused": bool, "int8_gemm": "hip" | None, "fallbacks": [...],
    ...}. Attention backends are outside this package; `attention_backend`
    is reported back unchanged.
    """
    if not torch.cuda.is_available():
        raise RuntimeError("the W8A8 path requires a GPU")
    result = {"attention_backend": attention_backend or "native", "fused": False,
              "int8_gemm": None, "fallbacks": []}
    device = torch.device("cuda", torch.cuda.current_device())
    with torch.inference_mode():
        try:
            from . import _lib
            probe = torch.empty(1, device=device)
            _lib.check_device(probe)
            if not _probe_gemm(device):
                raise RuntimeError("INT8 GEMM failed its exact numerical probe")
            result["int8_gemm"] = "hip"
            if not _probe_residual(device):
                raise RuntimeError("residual fusion failed its exact numerical probe")
            torch.cuda.synchronize(device)
            result["fused"] = True
            result["residual_quant_exact"] = True
        except Exception as error:  # reported, like the reference's probe
            if isinstance(error, torch.cuda.OutOfMemoryError):
                raise
            result["fallbacks"].append(f"gfx950 fusion unavailable: {error}")
    return result
