"""The fused block surface (model/fusion.py:12-162) on gfx950: fused_block's
output is bit-identical to the reference's unfused op sequence run through
this package's single kernels (which the other GPU tests pin to the oracle),
so the orchestration and the fused epilogues (residual + norm2 + quant, the
FFN-down gated residual in the GEMM) change nothing; the time-modulation
cache reuses tables per timestep key; a recoverable kernel failure falls
back to the native block."""
import numpy as np
import pytest
import torch

import blocks as toy
from lynnreal_omni_amd import fusion, kernels as k

pytestmark = pytest.mark.gpu

DIM, HEADS, INNER, TIME = 256, 2, 512, 128


def _attention(query, key, value, mask, processor):
    """Deterministic stand-in for the attention backend (outside this package)."""
    q, kk, v = (t.transpose(1, 2).float().contiguous() for t in (query, key, value))
    scores = torch.softmax(torch.matmul(q, kk.transpose(-1, -2).contiguous()) / q.shape[-1] ** 0.5, -1)
    return torch.matmul(scores, v).transpose(1, 2).to(query.dtype)


def _inputs(tokens=96, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(1, tokens, DIM, generator=g) * 2).bfloat16().cuda()
    temb = torch.randn(2, TIME, generator=g).cuda()               # two time rows
    idx = (torch.arange(tokens) * 2 // tokens).cuda()             # first half row 0, second row 1
    phase = torch.randn(tokens, DIM // HEADS, generator=g).cuda()
    return x, temb, idx, (phase.cos(), phase.sin())


def _block(seed=1):
    b = toy.Block(DIM, HEADS, INNER, TIME, torch.Generator().manual_seed(seed)).cuda().eval()
    # bf16 norms and adaLN projection; the Int8Linear scales stay fp32 (a
    # blanket .to(bfloat16) would convert them too, in the reference as here)
    for m in (b.norm1, b.norm2, b.attn.norm_q, b.attn.norm_k, b.adaln_proj):
        m.to(torch.bfloat16)
    return b


def _unfused(block, x, temb, idx, rotary):
    """model/fusion.py:61-98 (fused_quant path, reference residual order) step by step."""
    lin = block.adaln_proj.linear
    table = k.adaln_table(temb, lin.weight, lin.bias).view(-1, 6 * DIM)
    q, s = k._rms_adaln_quant_int8(x, block.norm1, table, idx, 0, 1)
    qkv = block.attn.to_qkv.forward_quantized(q, s, x.shape[:-1])
    query, key, value = (t.unflatten(-1, (HEADS, -1)) for t in qkv.chunk(3, dim=-1))
    qo, ko = k.qk_norm_rope(query, key, block.attn.norm_q.weight, block.attn.norm_k.weight, rotary,
                            block.attn.norm_q.eps)
    att = _attention(qo, ko, value, None, None).flatten(2, 3).type_as(qo)
    # with fused_quant the layers quantize through kernels.quantize_rows
    # (the Triton quantizer's semantics, model/int8.py:62-64)
    qa, sa = k.quantize_rows(att.reshape(-1, DIM))
    upd = block.attn.to_out[0].forward_quantized(qa, sa, att.shape[:-1])
    x1 = k._gated_residual(x, upd, table, idx, 2)
    q2, s2 = k._rms_adaln_quant_int8(x1, block.norm2, table, idx, 3, 4)
    proj = block.ff.net[0].proj.forward_quantized(q2, s2, x.shape[:-1])
    q3, s3 = k._swiglu_quant_int8(proj)
    y = block.ff.net[2].forward_quantized(q3, s3, proj.shape[:-1])
    return k._gated_residual(x1, y, table, idx, 5)


@torch.inference_mode()
def test_fused_block_equals_unfused_sequence():
    block = _block()
    x, temb, idx, rotary = _inputs()
    want = _unfused(block, x, temb, idx, rotary)
    report = fusion.enable_fusion(toy.Transformer([block]), fused_quant=True, attention=_attention)
    assert report["residual_ffn_norm_fused"] and report["qk_ordered_reduction"]
    got = block(x, temb, idx, rotary)
    assert got.dtype == torch.bfloat16 and torch.equal(got, want)


def _oracle_block(block, x, temb, idx, rotary):
    """The same block composed from the oracle's functions (model/fusion.py:61-98,
    fused_quant path), with the same attention stand-in fed the oracle's Q/K/V.
    Returns (qkv, first residual, block output) as bf16 bit patterns."""
    import torch.nn.functional as F
    from helpers import from_np, to_np
    from oracle import reference as ref

    def layer(lin):
        w_nk = lin.weight_int8.t().contiguous().cpu().numpy()
        return w_nk, to_np(lin.weight_scale.float()).reshape(-1), to_np(lin.bias)

    t = x.shape[-2]
    eps = block.norm1.eps
    lin = block.adaln_proj.linear
    # the adaLN kernel's fused silu equals torch's own GPU F.silu (test_gpu_adaln.py)
    table = ref.adaln_table(to_np(F.silu(temb).to(torch.bfloat16)), to_np(lin.weight), to_np(lin.bias))
    xi, ii = to_np(x), idx.cpu().numpy()
    q, s = ref.rms_adaln_quant(xi, to_np(block.norm1.weight), table, ii, 0, 1, eps)
    qkv = ref.linear(q, s, *layer(block.attn.to_qkv)).reshape(1, t, 3 * DIM)
    query, key, value = (qkv[..., i * DIM:(i + 1) * DIM].reshape(1, t, HEADS, DIM // HEADS) for i in range(3))
    cos, sin = (c.float().cpu().numpy() for c in rotary)
    qo, ko = ref.qk_norm_rope(query, key, to_np(block.attn.norm_q.weight), to_np(block.attn.norm_k.weight),
                              cos, sin, block.attn.norm_q.eps)
    dev = x.device
    att = _attention(from_np(qo, dev), from_np(ko, dev), from_np(np.ascontiguousarray(value), dev), None, None)
    qa, sa = ref.quantize_rows(to_np(att.flatten(2, 3)).reshape(t, DIM))
    upd = ref.linear(qa, sa, *layer(block.attn.to_out[0])).reshape(1, t, DIM)
    x1 = ref.gated_residual(xi, upd, table, ii, 2)
    q2, s2 = ref.rms_adaln_quant(x1, to_np(block.norm2.weight), table, ii, 3, 4, eps)
    proj = ref.linear(q2, s2, *layer(block.ff.net[0].proj))
    q3, s3 = ref.swiglu_quant(proj)
    y = ref.linear(q3, s3, *layer(block.ff.net[2])).reshape(1, t, DIM)
    return qkv, x1, ref.gated_residual(x1, y, table, ii, 5)


@torch.inference_mode()
def test_fused_block_against_oracle_chain():
    """fused_block against the block composed from the oracle's functions:
    the QKV projection and the first gated residual bit for bit (the unfused
    GPU sequence, which the fused block equals bit for bit, supplies those
    intermediates), the block output within the SwiGLU tolerance (the
    activation is within 2 bf16 ulp of the oracle's, so its int8 codes may
    move by one)."""
    from helpers import assert_bf16_close, to_np
    block = _block(11)
    x, temb, idx, rotary = _inputs(seed=12)
    want_qkv, want_x1, want_out = _oracle_block(block, x, temb, idx, rotary)
    lin = block.adaln_proj.linear
    table = k.adaln_table(temb, lin.weight, lin.bias).view(-1, 6 * DIM)
    q, s = k._rms_adaln_quant_int8(x, block.norm1, table, idx, 0, 1)
    qkv = block.attn.to_qkv.forward_quantized(q, s, x.shape[:-1])
    assert np.array_equal(to_np(qkv), want_qkv)
    query, key, value = (t.unflatten(-1, (HEADS, -1)) for t in qkv.chunk(3, dim=-1))
    qo, ko = k.qk_norm_rope(query, key, block.attn.norm_q.weight, block.attn.norm_k.weight, rotary,
                            block.attn.norm_q.eps)
    att = _attention(qo, ko, value, None, None).flatten(2, 3).type_as(qo)
    qa, sa = k.quantize_rows(att.reshape(-1, DIM))
    x1 = k._gated_residual(x, block.attn.to_out[0].forward_quantized(qa, sa, att.shape[:-1]), table, idx, 2)
    assert np.array_equal(to_np(x1), want_x1)
    unfused = _unfused(block, x, temb, idx, rotary)
    fusion.enable_fusion(toy.Transformer([block]), fused_quant=True, attention=_attention)
    got = block(x, temb, idx, rotary)
    assert torch.equal(got, unfused)
    # the north-star bar for bf16 outputs: max relative error <= 1e-2, cosine >= 0.9999
    assert_bf16_close(to_np(got), want_out, max_ulp=64, frac_exact=0.5, rel=1e-2, cos=0.9999, atol=1e-3)


@torch.inference_mode()
def test_fused_block_bf16_path():
    """fused_quant=False: modulated bf16 activations into the layers' own forward."""
    block = _block(2)
    x, temb, idx, rotary = _inputs(seed=3)
    lin = block.adaln_proj.linear
    table = k.adaln_table(temb, lin.weight, lin.bias).view(-1, 6 * DIM)
    h = k._rms_adaln(x, block.norm1, table, idx, 0, 1)
    query, key, value = (t.unflatten(-1, (HEADS, -1)) for t in block.attn.to_qkv(h).chunk(3, dim=-1))
    qo, ko = k.qk_norm_rope(query, key, block.attn.norm_q.weight, block.attn.norm_k.weight, rotary,
                            block.attn.norm_q.eps)
    upd = block.attn.to_out[0](_attention(qo, ko, value, None, None).flatten(2, 3))
    x1 = k._gated_residual(x, upd, table, idx, 2)
    proj = block.ff.net[0].proj(k._rms_adaln(x1, block.norm2, table, idx, 3, 4))
    want = k._gated_residual(x1, block.ff.net[2](k._swiglu(proj)), table, idx, 5)
    fusion.enable_fusion(toy.Transformer([block]), fused_quant=False, attention=_attention)
    assert torch.equal(block(x, temb, idx, rotary), want)


@torch.inference_mode()
def test_time_modulation_cache():
    blocks = [_block(4), _block(5)]
    model = toy.Transformer(blocks).eval()
    fusion.enable_fusion(model, fused_quant=True, attention=_attention)
    report = fusion.cache_time_modulation(model)
    assert report["maximum_entries_per_block"] == 16
    x, temb, idx, rotary = _inputs(seed=6)
    first = model(x, temb, idx, rotary, timestep=torch.tensor([0.5, 0.25]))
    cached = dict(blocks[0]._lynnreal_adaln_cache)
    assert len(cached) == 1
    again = model(x, temb, idx, rotary, timestep=torch.tensor([0.5, 0.25]))
    assert torch.equal(first, again) and len(blocks[0]._lynnreal_adaln_cache) == 1
    # the cached table is the one a fresh computation gives
    key = next(iter(cached))
    lin = blocks[0].adaln_proj.linear
    assert torch.equal(cached[key], k.adaln_table(temb, lin.weight, lin.bias).view(-1, 6 * DIM))
    for t in range(20):
        model(x, temb, idx, rotary, timestep=torch.tensor([float(t), 0.0]))
    assert len(blocks[0]._lynnreal_adaln_cache) == 16 and key not in blocks[0]._lynnreal_adaln_cache


@torch.inference_mode()
def test_guarded_block_falls_back_on_unsupported_kernel():
    block = _block(7)
    native = block.forward
    fusion.enable_fusion(toy.Transformer([block]), fused_quant=True, attention=_attention)
    x, temb, idx, _ = _inputs(seed=8)
    bad = torch.zeros(x.shape[1], 24, device="cuda")        # rotary_dim 24: not supported by the kernel
    with pytest.warns(RuntimeWarning, match="using native block"):
        out = block(x, temb, idx, (bad, bad))
    assert torch.equal(out, native(x, temb, idx, (bad, bad)))
    assert isinstance(block.attn.processor, toy.NativeProcessor)
    assert not block.attn.to_qkv.fused_ops


@torch.inference_mode()
def test_elementwise_block_forward():
    """model/elementwise_fusion.py:7-20: native norms and attention, the table,
    gated residuals and SwiGLU on this package's kernels."""
    from lynnreal_omni_amd import elementwise_fusion as ef
    block = _block(9)
    x, temb, idx, rotary = _inputs(seed=10)
    lin = block.adaln_proj.linear
    table = k.adaln_table(temb, lin.weight, lin.bias).view(-1, 6 * DIM)
    shift, scale, _, shift2, scale2, _ = table.chunk(6, dim=-1)
    h = block.norm1(x) * (1 + scale.index_select(0, idx)) + shift.index_select(0, idx)
    x1 = k._gated_residual(x, block.attn(h, rotary, None), table, idx, 2)
    h2 = block.norm2(x1) * (1 + scale2.index_select(0, idx)) + shift2.index_select(0, idx)
    want = k._gated_residual(x1, block.ff.net[2](k._swiglu(block.ff.net[0].proj(h2))), table, idx, 5)
    report = ef.enable_elementwise_fusion(toy.Transformer([block]).eval())
    assert report["swiglu"] and report["blocks"] == 1
    assert torch.equal(block(x, temb, idx, rotary), want)
