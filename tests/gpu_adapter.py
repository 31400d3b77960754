"""The HIP path behind the oracle's numpy API, so that the same checks
(tests/golden_check.py and the parity tests) run against both.

Every function copies numpy inputs to cuda:0, calls the drop-in module
function (lynnreal_omni_amd.kernels / int8_gemm), synchronizes and returns
numpy. bf16 arrays are uint16 bit patterns.
"""
from __future__ import annotations

import types

import numpy as np
import torch

from helpers import from_np, to_np
from lynnreal_omni_amd import int8_gemm, kernels

DEV = "cuda:0"


def _t(a, dtype=None):
    return from_np(np.asarray(a), DEV, dtype)


def _norm(w, eps):
    return types.SimpleNamespace(weight=_t(np.reshape(w, -1)), eps=eps)


def _done(*ts):
    torch.cuda.synchronize()
    out = tuple(to_np(t) for t in ts)
    return out if len(out) > 1 else out[0]


def quantize_rows(x):
    q, s = kernels.quantize_rows(_t(x))
    q, s = _done(q, s)
    return q, s.reshape(-1)


def int_mm(a, w_nk, *, tile=None):
    w = _t(w_nk)
    return _done(int8_gemm.int8_matmul_int32(_t(a), w.t(), tile=tile))


def dequant(acc, row_scale, col_scale, bias=None):
    return _done(kernels.int8_epilogue(_t(acc), _t(row_scale, torch.float32),
                                       _t(col_scale, torch.float32),
                                       None if bias is None else _t(bias)))


def linear(a_q, row_scale, w_nk, col_scale, bias=None, *, tile=None, **epilogue):
    w = _t(w_nk)
    extra = {k: (_t(v) if isinstance(v, np.ndarray) else v) for k, v in epilogue.items()}
    y = int8_gemm.int8_matmul(_t(a_q), w.t(), _t(row_scale, torch.float32),
                              _t(col_scale, torch.float32), None if bias is None else _t(bias),
                              tile=tile, **extra)
    return _done(y)


def gated_residual(x, u, table, indices, slot):
    return _done(kernels._gated_residual(_t(x), _t(u), _t(table), _t(indices), slot))


def rms_adaln(x, w, table, indices, shift_slot, scale_slot, eps):
    return _done(kernels._rms_adaln(_t(x), _norm(w, eps), _t(table), _t(indices), shift_slot,
                                    scale_slot))


def rms_adaln_quant(x, w, table, indices, shift_slot, scale_slot, eps):
    q, s = kernels._rms_adaln_quant_int8(_t(x), _norm(w, eps), _t(table), _t(indices), shift_slot,
                                         scale_slot)
    q, s = _done(q, s)
    return q, s.reshape(-1)


def residual_rms_quant(x, u, w, table, indices, eps):
    r, q, s = kernels.residual_rms_quant(_t(x), _t(u), _norm(w, eps), _t(table), _t(indices))
    r, q, s = _done(r, q, s)
    return r, q, s.reshape(-1)


def swiglu(p):
    return _done(kernels._swiglu(_t(p)))


def swiglu_quant(p):
    q, s = kernels._swiglu_quant_int8(_t(p))
    q, s = _done(q, s)
    return q, s.reshape(-1)


def gelu_tanh(x):
    return _done(kernels.gelu_tanh(_t(x)))


def gelu_quant(x):
    q, s = kernels._gelu_quant_int8(_t(x))
    q, s = _done(q, s)
    return q, s.reshape(-1)


module = types.SimpleNamespace(**{k: v for k, v in globals().items() if callable(v) and not k.startswith("_")})
