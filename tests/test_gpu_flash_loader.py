"""The Flash W8A8 loader (model/flash_int8.py:9-56) on the GPU: a synthetic
sharded folder loaded with device="cuda", gemm="triton" (the reference's
call), and every loaded projection, the fused Q/K/V included, run through
the HIP GEMM and compared with the C oracle bit for bit.

With fused_ops=True the layer quantizes its input with the HIP quantizer,
whose arithmetic is the oracle's (IEEE quotient). With fused_ops=False it
quantizes with torch's own GPU ops, as the reference does (model/int8.py:
66-67; torch's GPU division by the scalar 127 is a multiplication by its
reciprocal), and the GEMM is compared given those int8 rows and scales.
"""
import numpy as np
import pytest
import torch

from helpers import bf16_randn, to_np
from lynnreal_omni_amd import flash_int8
from lynnreal_omni_amd.int8 import Int8Linear, quantize_activations
from oracle import reference as ref
from test_flash_loader import BLOCKS, _make_folder, _Model

pytestmark = pytest.mark.gpu


def _oracle_linear(q, s, w_nk, scale, bias):
    return ref.linear(q, s.reshape(-1), w_nk, scale.reshape(-1), None if bias is None else to_np(bias))


@torch.inference_mode()
def test_loaded_flash_model_runs_the_hip_gemm(tmp_path):
    _, packed = _make_folder(tmp_path, seed=5)
    model = flash_int8.load_transformer(tmp_path, device="cuda", gemm="triton", model_factory=_Model)
    g = torch.Generator().manual_seed(6)
    checked = 0
    for b in range(BLOCKS):
        names = [f"attn.to_{p}" for p in "qkv"]
        qkv_parts = [packed[f"transformer_blocks.{b}.{n}"] for n in names]
        w_qkv = torch.cat([p[0] for p in qkv_parts]).numpy()
        s_qkv = torch.cat([p[1] for p in qkv_parts]).numpy()
        bias_qkv = torch.cat([p[2] if p[2] is not None else torch.zeros(p[0].shape[0], dtype=torch.bfloat16)
                              for p in qkv_parts])
        layers = {"attn.to_qkv": (w_qkv, s_qkv, bias_qkv)}
        for sub in ("attn.to_out.0", "ff.net.0.proj", "ff.net.2"):
            w, s, bias = packed[f"transformer_blocks.{b}.{sub}"]
            layers[sub] = (w.numpy(), s.numpy(), bias)
        for sub, (w, s, bias) in layers.items():
            layer = model.get_submodule(f"transformer_blocks.{b}.{sub}")
            assert isinstance(layer, Int8Linear) and layer.gemm == "triton"
            assert layer.weight_int8.is_cuda and layer.weight_int8.stride() == (1, layer.in_features)
            x = bf16_randn((3, 7, layer.in_features), g, outliers=0.02)
            xd = x.cuda()
            layer.fused_ops = True
            y = layer(xd)
            torch.cuda.synchronize()
            q, qs = ref.quantize_rows(to_np(x.reshape(-1, layer.in_features)))
            want = _oracle_linear(q, qs, w, s, bias)
            assert y.shape == (3, 7, layer.out_features)
            assert np.array_equal(to_np(y.reshape(-1, layer.out_features)), want), sub
            layer.fused_ops = False
            y = layer(xd)
            tq, ts = quantize_activations(xd.reshape(-1, layer.in_features))
            want = _oracle_linear(tq.cpu().numpy(), ts.cpu().numpy(), w, s, bias)
            assert np.array_equal(to_np(y.reshape(-1, layer.out_features)), want), sub
            checked += 1
    assert checked == 4 * BLOCKS
