"""Flash W8A8 loader (model/flash_int8.py:9-56) on a synthetic sharded folder (CPU).

The reference builds diffusers' MiniMaxH3Transformer3DModel, which is not
installed here; the tests pass a small module with the same submodule names
(transformer_blocks[i].attn.to_q/to_k/to_v/to_out.0, ff.net.0.proj, ff.net.2)
through `model_factory`. Everything else (checksums, shard index, module
replacement, Q/K/V fusion) is the loader's own logic.
"""
import hashlib
import json

import pytest
import torch
from torch import nn

from lynnreal_omni_amd import flash_int8
from lynnreal_omni_amd.int8 import Int8Linear

D, F, BLOCKS = 64, 128, 2


class _Proj(nn.Module):
    def __init__(self, i, o):
        super().__init__()
        self.proj = nn.Linear(i, o)


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.to_q, self.to_k, self.to_v = nn.Linear(D, D), nn.Linear(D, D, bias=False), nn.Linear(D, D)
        self.to_out = nn.ModuleList([nn.Linear(D, D), nn.Dropout(0.0)])
        self.fused_projections = False


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn = _Attn()
        self.ff = nn.Module()
        self.ff.net = nn.ModuleList([_Proj(D, F), nn.Dropout(0.0), nn.Linear(F, D)])
        self.norm_weight = nn.Parameter(torch.ones(D))


class _Model(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([_Block() for _ in range(config["blocks"])])
        self.proj_out = nn.Linear(D, 8)


QUANTIZED = [f"transformer_blocks.{b}.{m}" for b in range(BLOCKS)
             for m in ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0", "ff.net.0.proj", "ff.net.2")]


def _sha(path):
    return hashlib.sha256(path.read_bytes()).hexdigest()


def _make_folder(tmp_path, seed=0):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(seed)
    ref = _Model({"blocks": BLOCKS})
    tensors = {}
    for name, param in ref.state_dict().items():
        module = name.rsplit(".", 1)[0]
        if module in QUANTIZED:
            continue
        tensors[name] = torch.randn(param.shape, generator=g)
    packed = {}
    for name in QUANTIZED:
        lin = ref.get_submodule(name)
        w = torch.randint(-127, 128, (lin.out_features, lin.in_features), generator=g, dtype=torch.int8)
        s = torch.rand(lin.out_features, 1, generator=g) * 4e-3 + 1e-3
        tensors[name + ".weight_int8"] = w
        tensors[name + ".weight_scale"] = s
        if lin.bias is not None:
            tensors[name + ".bias"] = (0.02 * torch.randn(lin.out_features, generator=g)).bfloat16()
        packed[name] = (w, s, tensors.get(name + ".bias"))
    names = sorted(tensors)
    shards = {"model-00001-of-00002.safetensors": names[: len(names) // 2],
              "model-00002-of-00002.safetensors": names[len(names) // 2:]}
    weight_map = {}
    for shard, keys in shards.items():
        save_file({k: tensors[k].contiguous() for k in keys}, str(tmp_path / shard))
        weight_map.update({k: shard for k in keys})
    (tmp_path / "config.json").write_text(json.dumps({"blocks": BLOCKS}))
    (tmp_path / "quantization_config.json").write_text(json.dumps({"quantized_modules": QUANTIZED}))
    (tmp_path / "diffusion_pytorch_model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    checksums = {}
    for f in list(shards) + ["config.json", "quantization_config.json",
                             "diffusion_pytorch_model.safetensors.index.json"]:
        checksums[f] = {"sha256": _sha(tmp_path / f), "bytes": (tmp_path / f).stat().st_size}
    (tmp_path / "checksums.json").write_text(json.dumps(checksums))
    return tensors, packed


def _load(tmp_path, **kw):
    return flash_int8.load_transformer(tmp_path, device="cpu", gemm="torch", model_factory=_Model, **kw)


def test_loader_installs_packed_rows_and_fuses_qkv(tmp_path):
    tensors, packed = _make_folder(tmp_path)
    model = _load(tmp_path)
    assert not model.training
    for b, block in enumerate(model.transformer_blocks):
        attn = block.attn
        assert attn.to_q is None and attn.to_k is None and attn.to_v is None and attn.fused_projections
        qkv = attn.to_qkv
        assert isinstance(qkv, Int8Linear) and qkv.gemm == "torch"
        assert (qkv.in_features, qkv.out_features) == (D, 3 * D)
        names = [f"transformer_blocks.{b}.attn.to_{p}" for p in "qkv"]
        rows = torch.cat([packed[n][0] for n in names])
        assert qkv.weight_int8.stride() == (1, D) and torch.equal(qkv.weight_int8.t(), rows)
        assert torch.equal(qkv.weight_scale, torch.cat([packed[n][1] for n in names]).t())
        # to_k has no bias: its slice of the fused bias is zero (model/flash_int8.py:51-53)
        expect = torch.cat([packed[names[0]][2], torch.zeros(D, dtype=torch.bfloat16), packed[names[2]][2]])
        assert torch.equal(qkv.bias, expect)
        for sub in ("attn.to_out.0", "ff.net.0.proj", "ff.net.2"):
            layer = model.get_submodule(f"transformer_blocks.{b}.{sub}")
            w, s, bias = packed[f"transformer_blocks.{b}.{sub}"]
            assert isinstance(layer, Int8Linear)
            assert torch.equal(layer.weight_int8.t(), w) and torch.equal(layer.weight_scale, s.t())
            assert torch.equal(layer.bias, bias)
        assert torch.equal(block.norm_weight, tensors[f"transformer_blocks.{b}.norm_weight"])
    assert torch.equal(model.proj_out.weight, tensors["proj_out.weight"])


def test_loaded_layer_computes_the_w8a8_projection(tmp_path):
    _, packed = _make_folder(tmp_path)
    model = _load(tmp_path)
    layer = model.get_submodule("transformer_blocks.0.ff.net.2")
    x = torch.randn(5, F, generator=torch.Generator().manual_seed(3)).bfloat16()
    y = layer(x)
    w, s, bias = packed["transformer_blocks.0.ff.net.2"]
    xs = x.float()
    scale = xs.abs().amax(-1, keepdim=True).clamp_min(1e-8) / 127
    q = torch.clamp(torch.round(xs / scale), -127, 127)
    want = ((q @ w.float().t()) * scale * s.t() + bias.float()).bfloat16()
    assert y.dtype == torch.bfloat16 and torch.equal(y, want)


@pytest.mark.parametrize("tamper", ["shard", "metadata", "index", "incomplete"])
def test_loader_rejects_inconsistent_folders(tmp_path, tamper):
    _make_folder(tmp_path)
    if tamper == "shard":
        shard = tmp_path / "model-00001-of-00002.safetensors"
        data = bytearray(shard.read_bytes())
        data[-1] ^= 1
        shard.write_bytes(bytes(data))
        match = "shard checksum mismatch"
    elif tamper == "metadata":
        (tmp_path / "config.json").write_text(json.dumps({"blocks": BLOCKS, "x": 1}))
        match = "metadata checksum mismatch"
    else:
        index_path = tmp_path / "diffusion_pytorch_model.safetensors.index.json"
        index = json.loads(index_path.read_text())
        key = next(iter(index["weight_map"]))
        if tamper == "index":
            index["weight_map"]["not.a.tensor"] = index["weight_map"][key]
            match = "shard index mismatch"
        else:
            quant = json.loads((tmp_path / "quantization_config.json").read_text())
            quant["quantized_modules"] = quant["quantized_modules"][:-1]
            (tmp_path / "quantization_config.json").write_text(json.dumps(quant))
            match = "metadata checksum mismatch"
        index_path.write_text(json.dumps(index))
        checks = json.loads((tmp_path / "checksums.json").read_text())
        for f in ("diffusion_pytorch_model.safetensors.index.json", "quantization_config.json"):
            checks[f]["sha256"] = _sha(tmp_path / f)
        (tmp_path / "checksums.json").write_text(json.dumps(checks))
        if tamper == "incomplete":
            match = "Incomplete Flash model"
    with pytest.raises(ValueError, match=match):
        _load(tmp_path)
