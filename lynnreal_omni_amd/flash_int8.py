"""Load HF-sharded, trained Flash W8A8 tensors without requantization.

Drop-in for the reference's model/flash_int8.py:9-56 (`load_transformer`):
the same folder format, the same checks and error messages, the same
resulting modules (trained INT8 rows installed as Int8Linear layers, each
block's Q/K/V fused into one `to_qkv`).

Folder format (the reference's Flash release):
  config.json, quantization_config.json ({"quantized_modules": [names]}),
  diffusion_pytorch_model.safetensors.index.json ({"weight_map": {tensor: shard}}),
  checksums.json ({file: {"sha256": hex, "bytes": n}}), and the shards.
A quantized module `name` is stored as `name.weight_int8` (int8 [out, in]),
`name.weight_scale` (fp32 [out, 1]) and optionally `name.bias`; every other
tensor is an ordinary state-dict entry.

The loader works in three passes:
  1. read_checked verifies the metadata digests, then each shard's size and
     digest, and that each shard holds exactly the tensors the index assigns
     to it;
  2. the packed tensors of the quantized modules are taken out of the state
     dict as PackedRows; what remains must be exactly the model's float
     state (the model's keys minus the quantized modules' weight/bias);
  3. each block's Q/K/V rows are concatenated into one PackedRows before any
     layer is built, then every packed module becomes an Int8Linear and the
     float state is assigned.

The transformer class comes from diffusers in the reference
(MiniMaxH3Transformer3DModel, built on empty weights). Where diffusers is not
installed a caller passes `model_factory(config) -> nn.Module`.
"""
from __future__ import annotations

import collections
import hashlib
import json
import pathlib
from dataclasses import dataclass

import torch

from .int8 import Int8Linear

CONFIG = "config.json"
QUANT_CONFIG = "quantization_config.json"
SHARD_INDEX = "diffusion_pytorch_model.safetensors.index.json"
_QKV = ("to_q", "to_k", "to_v")


def sha256(path) -> str:
    """Hex SHA-256 of a file, read in 8 MiB blocks (model/weights.py:14-19)."""
    value = hashlib.sha256()
    with pathlib.Path(path).open("rb") as stream:
        for block in iter(lambda: stream.read(8 << 20), b""):
            value.update(block)
    return value.hexdigest()


class _Manifest:
    """A Flash folder and its checksums.json records."""

    def __init__(self, folder):
        self.folder = pathlib.Path(folder).resolve(strict=True)
        self.records = json.loads((self.folder / "checksums.json").read_text())

    def json(self, name):
        return json.loads((self.folder / name).read_text())

    def same_digest(self, name) -> bool:
        return sha256(self.folder / name) == self.records[name]["sha256"]

    def same_file(self, name) -> bool:
        # The size test is free and rejects most corrupt shards before hashing.
        size_ok = (self.folder / name).stat().st_size == self.records[name]["bytes"]
        return size_ok and self.same_digest(name)


def read_checked(folder, device="cpu"):
    """Verify a Flash folder against checksums.json and read its tensors.

    Returns (config, quantization_config, {tensor name: tensor}) with the
    tensors on `device`. Raises ValueError on a metadata digest, shard
    size/digest or shard index mismatch, with the reference's messages
    (model/flash_int8.py:14-32).
    """
    manifest = _Manifest(folder)
    for name in (CONFIG, QUANT_CONFIG, SHARD_INDEX):
        if not manifest.same_digest(name):
            raise ValueError("Flash metadata checksum mismatch: " + name)
    owned = collections.defaultdict(set)      # shard file -> the tensors the index puts there
    for tensor, shard in manifest.json(SHARD_INDEX)["weight_map"].items():
        owned[shard].add(tensor)
    from safetensors.torch import load_file
    tensors = {}
    for shard in sorted(owned):
        if not manifest.same_file(shard):
            raise ValueError("Flash shard checksum mismatch: " + shard)
        loaded = load_file(str(manifest.folder / shard), device=str(device))
        if loaded.keys() != owned[shard]:
            raise ValueError("Flash shard index mismatch")
        tensors.update(loaded)
    return manifest.json(CONFIG), manifest.json(QUANT_CONFIG), tensors


@dataclass
class PackedRows:
    """The stored form of one quantized projection."""
    weight: torch.Tensor            # int8 [out, in]
    scale: torch.Tensor             # fp32 [out, 1]
    bias: torch.Tensor | None       # bf16 [out] or None

    @classmethod
    def take(cls, tensors: dict, module: str) -> "PackedRows":
        """Remove `module`'s packed tensors from a state dict."""
        try:
            weight, scale = tensors.pop(module + ".weight_int8"), tensors.pop(module + ".weight_scale")
        except KeyError:
            raise ValueError(f"Incomplete Flash model: no packed rows for {module}") from None
        return cls(weight, scale, tensors.pop(module + ".bias", None))

    @classmethod
    def side_by_side(cls, parts: list["PackedRows"]) -> "PackedRows":
        """One projection whose outputs are the parts' outputs in order: the
        integer rows and their scales concatenated as stored (no
        requantization), biases likewise, zeros standing in for a missing
        bias when any part has one (model/flash_int8.py:47-55)."""
        bias = None
        if any(p.bias is not None for p in parts):
            bias = torch.cat([p.bias if p.bias is not None else
                              torch.zeros(p.weight.shape[0], dtype=torch.bfloat16, device=p.weight.device)
                              for p in parts])
        return cls(torch.cat([p.weight for p in parts]), torch.cat([p.scale for p in parts]), bias)

    def layer(self, gemm) -> Int8Linear:
        return Int8Linear.from_packed(self.weight, self.scale, self.bias, gemm)


def _diffusers_factory(config):
    from accelerate import init_empty_weights
    from diffusers import MiniMaxH3Transformer3DModel
    with init_empty_weights(include_buffers=False):
        return MiniMaxH3Transformer3DModel.from_config(config)


def _assign_module(model, dotted: str, layer) -> None:
    parent, _, leaf = dotted.rpartition(".")
    setattr(model.get_submodule(parent) if parent else model, leaf, layer)


def load_transformer(folder, device="cuda", gemm="triton", *, model_factory=None):
    """Build the Flash transformer with trained W8A8 projections (model/flash_int8.py:9-56)."""
    config, quant, state = read_checked(folder, device)
    model = (model_factory or _diffusers_factory)(config)
    packed = {name: PackedRows.take(state, name) for name in quant["quantized_modules"]}
    replaced = {f"{name}.{leaf}" for name in packed for leaf in ("weight", "bias")}
    float_state = set(model.state_dict()) - replaced
    if float_state != state.keys():
        raise ValueError("Incomplete Flash model: " + str(float_state ^ state.keys()))

    names = {module: name for name, module in model.named_modules()}
    fused = {}
    for block in model.transformer_blocks:
        prefix = names[block.attn] + "."
        if not all(prefix + p in packed for p in _QKV):
            raise ValueError(f"Flash block {names[block]} has no packed Q/K/V projections")
        fused[block.attn] = PackedRows.side_by_side([packed.pop(prefix + p) for p in _QKV])

    for name, rows in packed.items():
        _assign_module(model, name, rows.layer(gemm))
    result = model.load_state_dict(state, strict=False, assign=True)
    if result.unexpected_keys:
        raise ValueError(result.unexpected_keys)
    state.clear()
    for attn, rows in fused.items():
        attn.to_qkv = rows.layer(gemm)
        for part in _QKV:
            setattr(attn, part, None)
        attn.fused_projections = True
    return model.to(device).eval().requires_grad_(False)
