"""Host-side checks of the fused block surface (model/fusion.py:119-162) on the CPU:
validation that runs before any kernel."""
import pytest
import torch

import blocks as toy
from lynnreal_omni_amd import fusion


def _model(n=2):
    g = torch.Generator().manual_seed(0)
    return toy.Transformer([toy.Block(64, 2, 64, 32, g) for _ in range(n)]).eval()


def test_enable_fusion_rejects_strided_blocks():
    model = _model()
    model.transformer_blocks[1].h3_ffn_token_stride = 2
    with pytest.raises(ValueError, match="dense attention and FFN math"):
        fusion.enable_fusion(model)


def test_enable_fusion_installs_processors_and_reports():
    model = _model()
    report = fusion.enable_fusion(model, fused_quant=True)
    assert report["blocks"] == 2 and report["activation_quantization_fused"]
    for block in model.transformer_blocks:
        assert isinstance(block.attn.processor, fusion.FusedAttention)
        assert block._lynnreal_fused_quant and block.attn.to_qkv.fused_ops
        assert block.forward.__func__ is fusion.guarded_block
    # a second call keeps the first native forward/processor for the fallback
    native = model.transformer_blocks[0]._lynnreal_native_processor
    fusion.enable_fusion(model)
    assert model.transformer_blocks[0]._lynnreal_native_processor is native


def test_cache_time_modulation_needs_fused_blocks_and_frozen_inference():
    model = _model()
    with pytest.raises(ValueError, match="requires fused blocks"):
        fusion.cache_time_modulation(model)
    fusion.enable_fusion(model)
    fusion.cache_time_modulation(model)
    x = torch.zeros(1, 4, 64)
    with pytest.raises(ValueError, match="frozen inference"):
        model(x, torch.zeros(1, 32), torch.zeros(4, dtype=torch.long), None, timestep=torch.zeros(1))


def test_fused_attention_requires_padless_rotary():
    proc = fusion.FusedAttention(toy.NativeProcessor())
    with pytest.raises(ValueError, match="padless rotary layout"):
        proc(None, torch.zeros(1), None)
    with pytest.raises(ValueError, match="padless rotary layout"):
        proc(None, torch.zeros(1), (torch.zeros(1, 2, 3), torch.zeros(1, 2, 3)))
