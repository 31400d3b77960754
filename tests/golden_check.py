"""Checks an implementation of the path against the committed golden fixtures.

`impl` is a namespace with the oracle's numpy API (oracle.reference, or the
GPU adapter in tests/gpu_adapter.py): quantize_rows, int_mm, dequant,
rms_adaln, gated_residual, swiglu, gelu_tanh.
"""
from __future__ import annotations

import hashlib
import json
import pathlib

import numpy as np

from helpers import assert_bf16_close
from oracle import bf16

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def load_small():
    return dict(np.load(GOLDEN / "golden_small.npz", allow_pickle=False))


def load_kat():
    return json.loads((GOLDEN / "golden_kat.json").read_text())


def check_all(impl):
    g = load_small()
    for key in ("quant", "quant317"):
        q, s = impl.quantize_rows(g[f"{key}_x"])
        assert np.array_equal(q, g[f"{key}_q"]) and np.array_equal(s, g[f"{key}_s"]), key
    acc = impl.int_mm(g["lin_q"], g["lin_w"])
    assert np.array_equal(acc, g["lin_acc"])
    y = impl.dequant(acc, g["lin_s"], g["lin_ws"], g["lin_bias"])
    assert np.array_equal(y, g["lin_y"])
    r2 = impl.gated_residual(g["norm_x"], g["norm_u"], g["norm_table"], g["norm_idx"], 2)
    assert np.array_equal(r2, g["norm_r2"])
    r5 = impl.gated_residual(g["norm_x"], g["norm_u"], g["norm_table"], g["norm_idx"], 5)
    assert np.array_equal(r5, g["norm_r5"])
    # The fused norm reduces in its own defined order; the fixtures carry
    # torch's order (the reference's Triton semantics): tolerance.
    y01 = impl.rms_adaln(g["norm_x"], g["norm_w"], g["norm_table"], g["norm_idx"], 0, 1, 1e-6)
    assert_bf16_close(y01, g["norm_y01"], frac_exact=0.99)
    y34 = impl.rms_adaln(g["norm_r2"], g["norm_w"], g["norm_table"], g["norm_idx"], 3, 4, 1e-6)
    assert_bf16_close(y34, g["norm_y34"], frac_exact=0.99)
    q34, s34 = impl.quantize_rows(y34.reshape(-1, y34.shape[-1]))
    same_rows = (bf16.ulp_distance(y34, g["norm_y34"]).reshape(q34.shape[0], -1) == 0).all(axis=1)
    assert np.array_equal(q34[same_rows], g["norm_q34"][same_rows])
    assert np.abs(q34.astype(np.int32) - g["norm_q34"]).max() <= 1
    assert_bf16_close(impl.swiglu(g["swiglu_p"]), g["swiglu_y"], frac_exact=0.99)
    assert_bf16_close(impl.gelu_tanh(g["gelu_x"]), g["gelu_y"], frac_exact=0.99, atol=1e-4)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
