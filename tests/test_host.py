"""Host-side logic of the drop-in modules, on the CPU.

Covers the reference-compatible surface that does not need a GPU: argument
validation (model/int8_gemm.py:97-98, model/int8.py:29-30), tile mapping,
Int8Linear's buffers and torch backend (model/int8.py:6-68), the converter
(model/int8.py:71-104) and the error classifier (model/acceleration.py:49-56).
"""
import pathlib
import re
import types

import numpy as np
import pytest
import torch
from torch import nn

from helpers import bf16_randn, to_np
from lynnreal_omni_amd import _lib, acceleration, int8_gemm, int8_tma, kernels
from lynnreal_omni_amd.int8 import Int8Linear, quantize_transformer, quantize_weight
from oracle import reference as ref


def gen(seed):
    return torch.Generator().manual_seed(seed)


def test_tile_mapping():
    assert int8_gemm._tile_id(None) == 0
    assert int8_gemm._tile_id((128, 256, 128, 8, 3)) == 3
    assert int8_gemm._tile_id((128, 256, 128, 8, 4, 8)) == 3
    assert int8_gemm._tile_id((64, 128, 128, 4, 3, 0)) == 5
    assert int8_gemm._tile_id("generic") == 6
    assert int8_gemm._tile_id((256, 192, 128, 8, 3)) == 8
    for bad in ((32, 32, 64, 4, 2), (512, 512, 1, 1, 1), "fast", (1,)):
        with pytest.raises(ValueError):
            int8_gemm._tile_id(bad)


def test_autotune_cache_entries(monkeypatch, tmp_path):
    """The tile cache (model/int8_gemm.py:64-66,124-151 keeps one JSON file per
    key): every candidate survives the JSON round trip, anything else reads
    as absent, the file lives under LYNNREAL_AMD_CACHE_DIR, and autotuning is
    off unless LYNNREAL_AMD_AUTOTUNE asks for it."""
    import json
    for tile in int8_gemm._CANDIDATES:
        assert int8_gemm._decode(json.loads(json.dumps(int8_gemm._encode(tile)))) == tile
    for junk in ([32, 32], "fast", 7, {"bm": 256}, [256, 256, 128]):
        assert int8_gemm._decode(junk) is int8_gemm._MISSING
    monkeypatch.setenv("LYNNREAL_AMD_CACHE_DIR", str(tmp_path))
    key = ("lib", "7.2", "gpu", "gfx950", 256, 128, 256, 512, (1, 512), True, 0)
    path = int8_gemm._cache_file(key)
    assert path.parent == tmp_path and path.name.startswith("int8-") and path.suffix == ".json"
    assert int8_gemm._cache_file(key[:-1] + (1,)) != path
    monkeypatch.delenv("LYNNREAL_AMD_AUTOTUNE", raising=False)
    assert not int8_gemm._autotune_enabled()
    monkeypatch.setenv("LYNNREAL_AMD_AUTOTUNE", "0")
    assert not int8_gemm._autotune_enabled()
    monkeypatch.setenv("LYNNREAL_AMD_AUTOTUNE", "1")
    assert int8_gemm._autotune_enabled()
    assert int8_gemm._tile_id("auto") == int8_gemm._tile_id(None) == _lib.TILE_AUTO


def test_tile_ids_match_the_header():
    """Every LR_TILE_* of the C header has the same value in the Python
    bindings, and the named tiles map onto them."""
    header = pathlib.Path(__file__).resolve().parents[1] / "include" / "lynnreal_amd.h"
    ids = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define LR_TILE_(\w+) (\d+)", header.read_text())}
    assert len(ids) >= 14
    for name, value in ids.items():
        assert getattr(_lib, "TILE_" + name) == value, name
    assert int8_gemm._tile_id("persistent") == ids["256x256_PERSISTENT"]
    assert int8_gemm._tile_id("256x256_w4x2") == ids["256x256_W4x2"]
    assert int8_gemm._tile_id((192, 256, 128, 8, 3)) == ids["192x256"]


def test_int8_tma_default_tile_is_the_persistent_gemm(monkeypatch):
    """model/int8_tma.py:33-41's default tile runs the persistent GEMM; any
    other tile tuple is passed on to int8_matmul's tile mapping."""
    seen = []
    monkeypatch.setattr(int8_tma, "int8_matmul", lambda *args, **kw: seen.append(kw["tile"]))
    a = torch.zeros(4, 8, dtype=torch.int8)
    b = torch.zeros(3, 8, dtype=torch.int8).t()
    int8_tma.matmul(a, b, None, None)
    int8_tma.matmul(a, b, None, None, tile=(128, 128, 128, 8, 3))
    assert seen == ["persistent", (128, 128, 128, 8, 3)]
    with pytest.raises(ValueError, match="TMA requires"):
        int8_tma.matmul(a, b.contiguous(), None, None)


def test_int8_matmul_validation():
    a = torch.zeros(4, 8, dtype=torch.int8)
    b = torch.zeros(8, 3, dtype=torch.int8)
    rs, cs = torch.ones(4, 1), torch.ones(1, 3)
    with pytest.raises(ValueError, match="contiguous row-major"):
        int8_gemm.int8_matmul(a.float(), b, rs, cs)
    with pytest.raises(ValueError, match="contiguous row-major"):
        int8_gemm.int8_matmul(a.t(), b, rs, cs)
    with pytest.raises(ValueError, match="contiguous row-major"):
        int8_gemm.int8_matmul(a, b[:4], rs, cs)
    with pytest.raises(ValueError, match="GPU tensors"):
        int8_gemm.int8_matmul(a, b, rs, cs)


def test_kernel_wrappers_validate_before_launch():
    with pytest.raises(RuntimeError, match="not supported"):
        kernels.quantize_rows(torch.zeros(2, 8, dtype=torch.float64))
    with pytest.raises(ValueError, match="GPU tensors"):
        kernels.quantize_rows(torch.zeros(2, 8))                    # fp32 rows are supported
    with pytest.raises(ValueError, match="GPU tensors"):
        kernels.quantize_rows(torch.zeros(2, 8, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="not supported"):
        kernels._gated_residual(torch.zeros(1, 2, 8), torch.zeros(1, 2, 8, dtype=torch.bfloat16),
                                torch.zeros(1, 48, dtype=torch.bfloat16), torch.zeros(2), 2)
    with pytest.raises(ValueError, match="int32"):
        kernels.int8_epilogue(torch.zeros(2, 2), torch.ones(2), torch.ones(2), None)
    norm = types.SimpleNamespace(weight=torch.ones(8, dtype=torch.float32), eps=1e-6)
    with pytest.raises((ValueError, RuntimeError), match="GPU tensors|not supported"):
        kernels._rms_adaln(torch.zeros(1, 2, 8, dtype=torch.bfloat16), norm,
                           torch.zeros(1, 48, dtype=torch.bfloat16), torch.zeros(2), 0, 1)


def test_torch_matmul_matches_oracle():
    g = gen(1)
    a = torch.randint(-127, 128, (13, 64), dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (40, 64), dtype=torch.int8, generator=g)
    rs = torch.rand(13, 1, generator=g) / 127
    cs = torch.rand(1, 40, generator=g) / 127
    bias = (torch.randn(40, generator=g) * 0.02).bfloat16()
    y = int8_gemm._torch_matmul(a, w.t(), rs, cs, bias)
    expect = ref.dequant(ref.int_mm(a.numpy(), w.numpy()), rs.numpy(), cs.numpy(), to_np(bias))
    assert np.array_equal(to_np(y), expect)


def test_int8_linear_buffers_and_torch_backend():
    g = gen(2)
    src = nn.Linear(96, 72, bias=True).to(torch.bfloat16)
    with torch.no_grad():
        src.weight.copy_(torch.randn(72, 96, generator=g).bfloat16())
    layer = Int8Linear(src, gemm="torch")
    assert layer.weight_int8.shape == (96, 72) and layer.weight_int8.stride() == (1, 96)
    assert layer.weight_scale.shape == (1, 72) and layer.weight_scale.dtype == torch.float32
    assert layer.bias.dtype == torch.bfloat16 and layer.weight.dtype == torch.bfloat16
    assert layer.weight.numel() == 0
    assert (layer.in_features, layer.out_features, layer.fused_ops) == (96, 72, False)
    q, s = quantize_weight(src.weight)
    assert torch.equal(layer.weight_int8.t(), q) and torch.equal(layer.weight_scale.t(), s)
    x = bf16_randn((2, 5, 96), g, outliers=0.02)
    y = layer(x)
    assert y.shape == (2, 5, 72) and y.dtype == torch.bfloat16
    qx, sx = ref.quantize_rows(to_np(x.reshape(-1, 96)))
    expect = ref.linear(qx, sx, to_np(layer.weight_int8.t().contiguous()),
                        layer.weight_scale.numpy(), to_np(layer.bias))
    assert np.array_equal(to_np(y.reshape(-1, 72)), expect)
    with pytest.raises(ValueError):
        Int8Linear(src, gemm="cuda")


def test_from_packed_keeps_rows_exactly():
    g = gen(3)
    w = torch.randint(-127, 128, (40, 24), dtype=torch.int8, generator=g)
    s = torch.rand(40, 1, generator=g)
    layer = Int8Linear.from_packed(w, s)
    assert layer.gemm == "triton" and torch.equal(layer.weight_int8.t(), w)
    assert layer.weight_scale.shape == (1, 40) and layer.weight.dtype == torch.bfloat16
    with pytest.raises(ValueError, match="INT8"):
        Int8Linear.from_packed(w.float(), s)
    with pytest.raises(ValueError, match="INT8"):
        Int8Linear.from_packed(w, s.t())


def _fake_transformer(blocks=4, width=32, ffn=64):
    def block():
        attn = types.SimpleNamespace(
            to_q=nn.Linear(width, width), to_k=nn.Linear(width, width, bias=False),
            to_v=nn.Linear(width, width), to_out=[nn.Linear(width, width), nn.Identity()])
        ff = types.SimpleNamespace(net=[types.SimpleNamespace(proj=nn.Linear(width, ffn)), None,
                                        nn.Linear(ffn // 2, width)])
        return types.SimpleNamespace(attn=attn, ff=ff)
    return types.SimpleNamespace(transformer_blocks=[block() for _ in range(blocks)])


def test_quantize_transformer():
    t = _fake_transformer()
    b1 = t.transformer_blocks[1]
    q, k, v = b1.attn.to_q, b1.attn.to_k, b1.attn.to_v
    report = quantize_transformer(t, protected_edges=1)
    assert report["quantized_blocks"] == [1, 2] and report["quantized_linears"] == 8
    for i, b in enumerate(t.transformer_blocks):
        assert b.attn.to_q is None and b.attn.fused_projections
        assert isinstance(b.attn.to_qkv, Int8Linear) == (i in (1, 2))
    fused_w = torch.cat([q.weight, k.weight, v.weight])
    wq, ws = quantize_weight(fused_w)
    assert torch.equal(b1.attn.to_qkv.weight_int8.t(), wq)
    bias = b1.attn.to_qkv.bias.float()
    assert torch.equal(bias[32:64], torch.zeros(32))           # missing k bias -> zeros
    assert torch.equal(bias[:32], q.bias.detach().bfloat16().float())
    with pytest.raises(ValueError, match="unconverted"):
        quantize_transformer(t)
    with pytest.raises(ValueError, match="protected"):
        quantize_transformer(_fake_transformer(blocks=2), protected_edges=1)


def test_optional_kernel_failure():
    ok = acceleration.optional_kernel_failure
    assert ok(RuntimeError("lr_int8_gemm: int8_gemm: too many tiles (not supported)"))
    assert ok(RuntimeError("no kernel image is available"))
    assert not ok(RuntimeError("illegal memory access"))
    assert not ok(ValueError("bad shape"))
    assert not ok(torch.cuda.OutOfMemoryError("not supported"))


def test_int8_tma_entry_checks_layout():
    from lynnreal_omni_amd import int8_tma
    a = torch.zeros(4, 64, dtype=torch.int8)
    w = torch.zeros(32, 64, dtype=torch.int8)
    s = torch.ones(4)
    with pytest.raises(ValueError, match="TMA requires"):
        int8_tma.matmul(a, w.t().contiguous(), s, torch.ones(32))      # stride (32, 1), not (1, K)
    with pytest.raises(ValueError, match="TMA requires"):
        int8_tma.matmul(a.float(), w.t(), s, torch.ones(32))
