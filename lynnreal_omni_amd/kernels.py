"""Fused row/element-wise kernels of the W8A8 path, on gfx950 HIP.

Same names, signatures and output allocation as the reference's Triton module
model/kernels.py; each function launches one kernel of liblynnreal_amd.so on
the caller's current stream. Outputs are allocated with torch.empty on the
input's device (the reference's ownership rule); inputs are made contiguous
and never modified.

Arithmetic (all fp32 with the reference's bf16 rounding points):
  quantize_rows        s = max(absmax, 1e-8)/127; q = clamp(rint(x/s), +-127)
                       (the torch path, model/int8.py:66-67)
  int8_epilogue        bf16((acc*as)*ws + bias)               kernels.py:27-38
  _rms_adaln(_quant)   RMSNorm*gamma -> bf16, *bf16(1+scale) -> bf16,
                       +shift -> bf16 (-> INT8)               kernels.py:48-128
  residual_rms_quant   x' = bf16(x + bf16(gate2*u)), then slots 3/4
                                                              kernels.py:405-419
  _gated_residual      bf16(x + bf16(gate*u))                 kernels.py:131-153
  _swiglu(_quant)      bf16(v * bf16(g*sigmoid(g))) (-> INT8)  kernels.py:156-185
  gelu_tanh            bf16(gelu_tanh(x))  (new: the benchmark FFN activation)
  _gelu_quant_int8     quantize_rows(gelu_tanh(x)) in one pass (new)
  qk_norm_rope         per-head RMSNorm of Q/K -> bf16, RoPE with bf16 products
                                                              kernels.py:187-257,345-402
  adaln_table          bf16(bf16(silu(temb)) @ W^T + bias)     fusion.py:68-69

The RMSNorm sum of squares uses one fixed reduction order (documented in
include/lynnreal_amd.h) and an IEEE 1/sqrt, so the bf16 outputs reproduce a
CPU restatement exactly; against the reference's Triton tree-sum and
approximate rsqrt they agree to a bf16 ulp.
"""
from __future__ import annotations

import torch

from . import _lib


def _bf16(t: torch.Tensor, what: str) -> torch.Tensor:
    """t contiguous, or RuntimeError("... not supported") for another dtype:
    these kernels read bfloat16, and the error is one that
    acceleration.optional_kernel_failure lets a caller fall back from (the
    reference's Triton kernels load any float dtype, model/kernels.py:64,100,146)."""
    if t.dtype != torch.bfloat16:
        raise RuntimeError(f"{what}: dtype {t.dtype} is not supported by the HIP kernel (bfloat16 only)")
    return t.contiguous()


def _norm_args(source, norm, table, indices):
    source = _bf16(source, "source")
    _lib.check_device(source)
    weight = getattr(norm, "weight", None)
    if weight is None:
        raise ValueError("norm must have a weight")
    _lib.same_device(source, **{"norm.weight": weight}, table=table, indices=indices)
    weight = _bf16(weight, "norm.weight")
    table = _bf16(table, "table")
    indices = indices.reshape(-1).contiguous()
    if indices.dtype != torch.int64:
        indices = indices.to(torch.int64)
    hidden = source.shape[-1]
    sequence = source.shape[-2] if source.dim() >= 2 else 1
    if weight.numel() != hidden:
        raise ValueError(f"norm.weight has {weight.numel()} elements, expected {hidden}")
    if indices.numel() < sequence:
        raise ValueError(f"indices has {indices.numel()} entries for a sequence of {sequence}")
    width = table.shape[-1]
    table_rows = table.numel() // width if width else 0
    return source, weight, table, indices, hidden, sequence, width, table_rows


_QUANT_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
                 torch.float32: _lib.DTYPE_F32}


def quantize_rows(value):
    """Per-row symmetric INT8 quantizer (model/kernels.py:19-24) for bf16,
    fp16 or fp32 rows (the Triton kernel loads any float row as fp32)."""
    rows, width = value.shape
    dtype = _QUANT_DTYPES.get(value.dtype)
    if dtype is None:
        raise RuntimeError(f"value: dtype {value.dtype} is not supported by the HIP quantizer")
    value = value.contiguous()
    _lib.check_device(value)
    output = torch.empty_like(value, dtype=torch.int8)
    scales = torch.empty(rows, 1, device=value.device, dtype=torch.float32)
    if dtype == _lib.DTYPE_BF16:
        _lib.call("lr_quantize_rows", value.data_ptr(), rows, width, output.data_ptr(),
                  scales.data_ptr(), _lib.stream(value))
    else:
        _lib.call("lr_quantize_rows_typed", value.data_ptr(), dtype, rows, width, output.data_ptr(),
                  scales.data_ptr(), _lib.stream(value))
    return output, scales


def int8_epilogue(accumulator, activation_scale, weight_scale, bias):
    """INT32 -> bf16 dequant epilogue (model/kernels.py:41-46)."""
    if accumulator.dtype != torch.int32:
        raise ValueError("accumulator must be int32")
    accumulator = accumulator.contiguous()
    _lib.check_device(accumulator)
    _lib.same_device(accumulator, activation_scale=activation_scale, weight_scale=weight_scale,
                     bias=bias)
    width = accumulator.shape[-1]
    rows = accumulator.numel() // width if width else 0
    a_scale = activation_scale.reshape(-1).float().contiguous()
    w_scale = weight_scale.reshape(-1).float().contiguous()
    if a_scale.numel() != rows or w_scale.numel() != width:
        raise ValueError("scale shapes do not match the accumulator")
    if bias is not None:
        bias = _bf16(bias.reshape(-1), "bias")
        if bias.numel() != width:
            raise ValueError("bias shape does not match the accumulator")
    output = torch.empty_like(accumulator, dtype=torch.bfloat16)
    _lib.call("lr_int8_epilogue", accumulator.data_ptr(), a_scale.data_ptr(), w_scale.data_ptr(),
              _lib.ptr(bias), output.data_ptr(), rows, width, _lib.stream(accumulator))
    return output


def _rms_adaln(source, norm, table, indices, shift_slot, scale_slot):
    """RMSNorm + adaLN modulate, bf16 out (model/kernels.py:260-272)."""
    source, weight, table, indices, hidden, sequence, width, table_rows = _norm_args(
        source, norm, table, indices)
    rows = source.numel() // hidden
    output = torch.empty_like(source)
    _lib.call("lr_rms_adaln", source.data_ptr(), weight.data_ptr(), table.data_ptr(),
              indices.data_ptr(), output.data_ptr(), rows, sequence, hidden, table_rows, width,
              int(shift_slot), int(scale_slot), float(norm.eps), _lib.stream(source))
    return output


def _rms_adaln_quant_int8(source, norm, table, indices, shift_slot, scale_slot):
    """RMSNorm + adaLN modulate + INT8 quant (model/kernels.py:275-289)."""
    source, weight, table, indices, hidden, sequence, width, table_rows = _norm_args(
        source, norm, table, indices)
    rows = source.numel() // hidden
    output = torch.empty((rows, hidden), device=source.device, dtype=torch.int8)
    scales = torch.empty((rows, 1), device=source.device, dtype=torch.float32)
    _lib.call("lr_rms_adaln_quant", source.data_ptr(), weight.data_ptr(), table.data_ptr(),
              indices.data_ptr(), output.data_ptr(), scales.data_ptr(), rows, sequence, hidden,
              table_rows, width, int(shift_slot), int(scale_slot), float(norm.eps),
              _lib.stream(source))
    return output, scales


def residual_rms_quant(source, update, norm, table, indices):
    """Gated residual (slot 2) fused with norm/modulate (slots 3, 4) and INT8
    quant (model/kernels.py:405-419)."""
    source, weight, table, indices, hidden, sequence, width, table_rows = _norm_args(
        source, norm, table, indices)
    update = _bf16(update, "update")
    _lib.same_device(source, update=update)
    if update.shape != source.shape:
        raise ValueError("update must have the shape of source")
    rows = source.numel() // hidden
    residual = torch.empty_like(source)
    quantized = torch.empty((rows, hidden), device=source.device, dtype=torch.int8)
    scales = torch.empty((rows, 1), device=source.device, dtype=torch.float32)
    _lib.call("lr_residual_rms_quant", source.data_ptr(), update.data_ptr(), weight.data_ptr(),
              table.data_ptr(), indices.data_ptr(), residual.data_ptr(), quantized.data_ptr(),
              scales.data_ptr(), rows, sequence, hidden, table_rows, width, float(norm.eps),
              _lib.stream(source))
    return residual, quantized, scales


def _gated_residual(residual, update, table, indices, gate_slot):
    """residual + gate * update with per-token gate (model/kernels.py:292-304)."""
    residual = _bf16(residual, "residual")
    _lib.check_device(residual)
    _lib.same_device(residual, update=update, table=table, indices=indices)
    update = _bf16(update, "update")
    if update.shape != residual.shape:
        raise ValueError("update must have the shape of residual")
    table = _bf16(table, "table")
    indices = indices.reshape(-1).contiguous()
    if indices.dtype != torch.int64:
        indices = indices.to(torch.int64)
    hidden = residual.shape[-1]
    sequence = residual.shape[-2] if residual.dim() >= 2 else 1
    if indices.numel() < sequence:
        raise ValueError(f"indices has {indices.numel()} entries for a sequence of {sequence}")
    width = table.shape[-1]
    rows = residual.numel() // hidden
    output = torch.empty_like(residual)
    _lib.call("lr_gated_residual", residual.data_ptr(), update.data_ptr(), table.data_ptr(),
              indices.data_ptr(), output.data_ptr(), rows, sequence, hidden,
              table.numel() // width if width else 0, width, int(gate_slot),
              _lib.stream(residual))
    return output


def _swiglu(projected):
    """SwiGLU of [.., 2I] -> [.., I] (model/kernels.py:307-315)."""
    projected = _bf16(projected, "projected")
    _lib.check_device(projected)
    inner = projected.shape[-1] // 2
    rows = projected.numel() // projected.shape[-1] if projected.shape[-1] else 0
    output = torch.empty((*projected.shape[:-1], inner), device=projected.device,
                         dtype=projected.dtype)
    _lib.call("lr_swiglu", projected.data_ptr(), output.data_ptr(), rows, inner,
              _lib.stream(projected))
    return output


def _swiglu_quant_int8(projected):
    """SwiGLU + INT8 quant (model/kernels.py:318-328)."""
    projected = _bf16(projected, "projected")
    _lib.check_device(projected)
    inner = projected.shape[-1] // 2
    rows = projected.numel() // projected.shape[-1]
    output = torch.empty((rows, inner), device=projected.device, dtype=torch.int8)
    scales = torch.empty((rows, 1), device=projected.device, dtype=torch.float32)
    _lib.call("lr_swiglu_quant", projected.data_ptr(), output.data_ptr(), scales.data_ptr(), rows,
              inner, _lib.stream(projected))
    return output, scales


def gelu_tanh(value):
    """Element-wise GELU (tanh approximation), bf16 in and out."""
    value = _bf16(value, "value")
    _lib.check_device(value)
    output = torch.empty_like(value)
    _lib.call("lr_gelu_tanh", value.data_ptr(), output.data_ptr(), value.numel(),
              _lib.stream(value))
    return output


def _gelu_quant_int8(value):
    """GELU-tanh + INT8 quant of [.., width] rows -> (int8 [rows, width],
    fp32 [rows, 1]): quantize_rows(gelu_tanh(value)) in one pass, the GELU
    counterpart of _swiglu_quant_int8 (model/kernels.py:318-328)."""
    value = _bf16(value, "value")
    _lib.check_device(value)
    width = value.shape[-1]
    rows = value.numel() // width if width else 0
    value = value.reshape(rows, width).contiguous()
    output = torch.empty((rows, width), device=value.device, dtype=torch.int8)
    scales = torch.empty((rows, 1), device=value.device, dtype=torch.float32)
    _lib.call("lr_gelu_quant", value.data_ptr(), output.data_ptr(), scales.data_ptr(), rows, width,
              _lib.stream(value))
    return output, scales


def qk_norm_rope(query, key, query_weight, key_weight, rotary_emb, eps):
    """Per-head RMSNorm of Q and K fused with RoPE (model/fusion.py:35-52).

    query, key: bf16 [batch, sequence, heads, head_dim] with contiguous heads
    (views into a fused QKV tensor are fine); query_weight, key_weight: bf16
    [head_dim] (attn.norm_q/norm_k weights); rotary_emb: (cos, sin), each
    [sequence, rotary_dim] (rounded to bf16 in the kernel, as the reference
    does). Returns new contiguous (q_out, k_out) like query. Both of the
    reference's kernels (full-width paired RoPE and partial RoPE) are this one
    launch; rotary_dim == 0 gives the bare RMSNorm.
    """
    cos, sin = rotary_emb
    rotary_dim = cos.shape[-1]
    if query.dim() != 4 or key.shape != query.shape:
        raise ValueError("query and key must be [batch, sequence, heads, head_dim] of one shape")
    head_dim = query.shape[-1]
    if rotary_dim > head_dim or rotary_dim % 2:
        raise ValueError("rotary dimensions must be even and fit the attention head")
    for name, t in (("query", query), ("key", key)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    _lib.check_device(query)
    _lib.same_device(query, key=key, query_weight=query_weight, key_weight=key_weight, cos=cos, sin=sin)
    if query_weight.numel() != head_dim or key_weight.numel() != head_dim:
        raise ValueError(f"query/key norm weights must have head_dim={head_dim} entries, got "
                         f"{query_weight.numel()} and {key_weight.numel()}")

    def rows(t):
        # Element (b, t, h, d) must sit at b*S*token_stride + t*token_stride + h*head_stride + d.
        if t.stride(3) != 1 or t.stride(0) != t.shape[1] * t.stride(1):
            t = t.contiguous()
        return t

    query, key = rows(query), rows(key)
    query_weight = _bf16(query_weight.reshape(-1), "query_weight")
    key_weight = _bf16(key_weight.reshape(-1), "key_weight")
    if cos.shape != sin.shape:
        raise ValueError("cos and sin tables must have one shape")
    batch, sequence, heads, _ = query.shape
    if rotary_dim:
        cos = cos.to(torch.float32).reshape(-1, rotary_dim).contiguous()
        sin = sin.to(torch.float32).reshape(-1, rotary_dim).contiguous()
        if cos.shape[0] < sequence:
            raise ValueError(f"rotary tables have {cos.shape[0]} positions for {sequence} tokens")
    q_out = torch.empty(query.shape, device=query.device, dtype=query.dtype)
    k_out = torch.empty_like(q_out)
    _lib.call("lr_qk_norm_rope", query.data_ptr(), key.data_ptr(), query_weight.data_ptr(),
              key_weight.data_ptr(), cos.data_ptr() if rotary_dim else None,
              sin.data_ptr() if rotary_dim else None, q_out.data_ptr(),
              k_out.data_ptr(), batch, sequence, heads, query.stride(1), query.stride(2),
              key.stride(1), key.stride(2), head_dim, rotary_dim, float(eps), _lib.stream(query))
    return q_out, k_out


def adaln_table(temb, weight, bias=None, *, silu=True):
    """The adaLN table linear(F.silu(temb).to(bf16)) (model/fusion.py:68-69).

    temb: fp32 or bf16 [..., in_features]; weight: bf16 [out_features,
    in_features] (nn.Linear.weight); bias: bf16 [out_features] or None.
    Returns bf16 [rows, out_features], rows = temb.numel() // in_features.
    silu=False skips the activation (bf16(temb) is used as is).
    """
    if temb.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"temb must be float32 or bfloat16, got {temb.dtype}")
    weight = _bf16(weight, "weight")
    _lib.check_device(weight)
    _lib.same_device(weight, temb=temb, bias=bias)
    out_features, in_features = weight.shape
    if temb.shape[-1] != in_features:
        raise ValueError(f"temb has {temb.shape[-1]} features, the weight expects {in_features}")
    temb = temb.reshape(-1, in_features).contiguous()
    if bias is not None:
        bias = _bf16(bias.reshape(-1), "bias")
        if bias.numel() != out_features:
            raise ValueError(f"bias has {bias.numel()} entries, expected {out_features}")
    out = torch.empty(temb.shape[0], out_features, device=weight.device, dtype=torch.bfloat16)
    _lib.call("lr_adaln_table", temb.data_ptr(), int(temb.dtype == torch.bfloat16), int(bool(silu)),
              weight.data_ptr(), _lib.ptr(bias), out.data_ptr(), temb.shape[0], in_features,
              out_features, _lib.stream(weight))
    return out
