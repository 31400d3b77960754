"""Load HF-sharded, trained Flash W8A8 tensors without requantization.

Drop-in for the reference's model/flash_int8.py:9-56 (`load_transformer`):
the same folder layout, checks, module replacement and Q/K/V fusion.

Folder layout (the reference's Flash release format):
  config.json, quantization_config.json ({"quantized_modules": [names]}),
  diffusion_pytorch_model.safetensors.index.json ({"weight_map": {tensor: shard}}),
  checksums.json ({file: {"sha256": hex, "bytes": n}}), and the shards.
A quantized module `name` is stored as `name.weight_int8` (int8 [out, in]),
`name.weight_scale` (fp32 [out, 1]) and optionally `name.bias`; every other
tensor is an ordinary state-dict entry.

The transformer class comes from diffusers in the reference
(MiniMaxH3Transformer3DModel, built on empty weights). Where diffusers is not
installed a caller passes `model_factory(config) -> nn.Module` instead; the
loading logic is the same either way.
"""
from __future__ import annotations

import hashlib
import json
import pathlib

import torch

from .int8 import Int8Linear

_METADATA = ("config.json", "quantization_config.json",
             "diffusion_pytorch_model.safetensors.index.json")


def sha256(path) -> str:
    """Hex SHA-256 of a file, read in 8 MiB blocks (model/weights.py:14-19)."""
    value = hashlib.sha256()
    with pathlib.Path(path).open("rb") as stream:
        for block in iter(lambda: stream.read(8 << 20), b""):
            value.update(block)
    return value.hexdigest()


def _diffusers_factory(config):
    from accelerate import init_empty_weights
    from diffusers import MiniMaxH3Transformer3DModel
    with init_empty_weights(include_buffers=False):
        return MiniMaxH3Transformer3DModel.from_config(config)


def read_checked(folder, device="cpu"):
    """Verify metadata and shards against checksums.json and read them.

    Returns (config, quantization_config, {tensor name: tensor}) with the
    tensors on `device`. Raises ValueError on any checksum, size or index
    mismatch, with the reference's messages (model/flash_int8.py:14-32).
    """
    folder = pathlib.Path(folder).resolve(strict=True)
    checksums = json.loads((folder / "checksums.json").read_text())
    for name in _METADATA:
        if sha256(folder / name) != checksums[name]["sha256"]:
            raise ValueError("Flash metadata checksum mismatch: " + name)
    config = json.loads((folder / "config.json").read_text())
    quant = json.loads((folder / "quantization_config.json").read_text())
    index = json.loads((folder / _METADATA[2]).read_text())["weight_map"]
    from safetensors.torch import load_file
    tensors = {}
    for filename in sorted(set(index.values())):
        path = folder / filename
        if path.stat().st_size != checksums[filename]["bytes"] or sha256(path) != checksums[filename]["sha256"]:
            raise ValueError("Flash shard checksum mismatch: " + filename)
        shard = load_file(str(path), device=str(device))
        if set(shard) != {k for k, v in index.items() if v == filename}:
            raise ValueError("Flash shard index mismatch")
        tensors.update(shard)
    return config, quant, tensors


def fuse_qkv(model, gemm="triton"):
    """Replace each block's to_q/to_k/to_v by one Int8Linear `to_qkv`.

    The integer rows and their scales are concatenated as stored (no
    requantization), biases likewise with zeros for a missing one
    (model/flash_int8.py:48-55). The fused GEMM then runs N = 3 * hidden.
    """
    for block in model.transformer_blocks:
        attn = block.attn
        parts = [attn.to_q, attn.to_k, attn.to_v]
        bias = None
        if any(p.bias is not None for p in parts):
            bias = torch.cat([p.bias if p.bias is not None else p.weight.new_zeros(p.out_features)
                              for p in parts])
        attn.to_qkv = Int8Linear.from_packed(torch.cat([p.weight_int8.t() for p in parts]),
                                             torch.cat([p.weight_scale.t() for p in parts]), bias, gemm)
        attn.to_q = attn.to_k = attn.to_v = None
        attn.fused_projections = True
    return model


def load_transformer(folder, device="cuda", gemm="triton", *, model_factory=None):
    """Build the Flash transformer with trained W8A8 projections (model/flash_int8.py:9-56)."""
    config, quant, pending = read_checked(folder, device)
    model = (model_factory or _diffusers_factory)(config)
    remaining = set(model.state_dict())
    for name in quant["quantized_modules"]:
        weight = pending.pop(name + ".weight_int8")
        scale = pending.pop(name + ".weight_scale")
        bias = pending.pop(name + ".bias", None)
        layer = Int8Linear.from_packed(weight, scale, bias, gemm)
        parent, _, key = name.rpartition(".")
        setattr(model.get_submodule(parent), key, layer)
        remaining.difference_update({name + ".weight", name + ".bias"})
    if set(pending) != remaining:
        raise ValueError("Incomplete Flash model: " + str(set(pending) ^ remaining))
    result = model.load_state_dict(pending, strict=False, assign=True)
    if result.unexpected_keys:
        raise ValueError(result.unexpected_keys)
    del pending
    fuse_qkv(model, gemm)
    return model.to(device).eval().requires_grad_(False)
