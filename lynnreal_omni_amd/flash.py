"""Flash token selection on gfx950: drop-in for the reference's model/flash.py.

Flash runs its middle blocks on a spatially subsampled token set:

  spatial_layout   which rows the middle blocks keep (every `stride`-th
                   distinct h and w coordinate of the video rows, plus the
                   last, and every non-video row), and for every row the
                   kept row it is restored from (a dropped video row takes
                   its nearest kept row of the same time step)
                   model/flash.py:6-33
  configure_flash  forward hooks: gather the kept rows before the first
                   compressed block, restore full + gain * (current - input)
                   through the inverse map before the first full block
                   model/flash.py:36-96

The row gather, the fused restore and the nearest-anchor search are HIP
kernels (lr_gather_rows, lr_flash_restore, lr_flash_nearest_anchor); the
alphabet/mask bookkeeping of the layout is O(tokens) torch plumbing on the
same device. Every output is a new tensor on the input's device, launched on
the caller's current stream; nothing falls back to the CPU.
"""
from __future__ import annotations

import inspect
import math

import torch

from . import _lib

VIDEO_TAG = 0


def gather_rows(source: torch.Tensor, index: torch.Tensor, dim: int) -> torch.Tensor:
    """source.index_select(dim, index) through lr_gather_rows.

    Any dtype; the result is contiguous. `index` entries must lie in
    [0, source.shape[dim]) (the kernel clamps others instead of reading
    outside the tensor).
    """
    _lib.check_device(source)
    if source.dim() == 0:
        raise ValueError("gather_rows needs a tensor with at least one dimension")
    dim = dim % source.dim()
    source = source.contiguous()
    index = index.reshape(-1).to(device=source.device, dtype=torch.int64).contiguous()
    shape = list(source.shape)
    outer, rows, inner = math.prod(shape[:dim]), shape[dim], math.prod(shape[dim + 1:])
    shape[dim] = index.numel()
    out = torch.empty(shape, dtype=source.dtype, device=source.device)
    _lib.call("lr_gather_rows", source.data_ptr(), index.data_ptr(), out.data_ptr(), outer, rows,
              index.numel(), inner * source.element_size(), _lib.stream(source))
    return out


def restore(full: torch.Tensor, current: torch.Tensor, input: torch.Tensor,
            inverse: torch.Tensor, gain: float = 1.0) -> torch.Tensor:
    """full + ((current - input) * gain).index_select(1, inverse), bf16, one pass.

    full [B, T, D]; current, input [B, T', D]; inverse int64 [T] in [0, T').
    Each bf16 operation rounds once, as the reference's tensor expression
    (model/flash.py:83-84) does.
    """
    _lib.check_device(full)
    for name, t in (("full", full), ("current", current), ("input", input)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
        if t.dim() < 2:
            raise ValueError(f"{name} must be [batch, tokens, ...]")
    if current.shape != input.shape:
        raise ValueError("current and input must have one shape")
    if (full.shape[0] != current.shape[0] or full.shape[2:] != current.shape[2:]
            or inverse.numel() != full.shape[1]):
        raise ValueError("restore: full, current and inverse do not describe one layout")
    full, current, input = full.contiguous(), current.contiguous(), input.contiguous()
    inverse = inverse.reshape(-1).to(device=full.device, dtype=torch.int64).contiguous()
    out = torch.empty_like(full)
    width = math.prod(full.shape[2:])
    _lib.call("lr_flash_restore", full.data_ptr(), current.data_ptr(), input.data_ptr(),
              inverse.data_ptr(), out.data_ptr(), full.shape[0], full.shape[1], current.shape[1],
              width, float(gain), _lib.stream(full))
    return out


def _retained(values: torch.Tensor, stride: int) -> torch.Tensor:
    """Every stride-th distinct value in increasing order, and always the largest."""
    alphabet = torch.unique(values, sorted=True)
    picked = alphabet[::stride]
    if picked[-1] != alphabet[-1]:
        picked = torch.cat((picked, alphabet[-1:]))
    return picked


def spatial_layout(positions: torch.Tensor, tags: torch.Tensor, stride: int = 2):
    """(keep, inverse) of the Flash selection (model/flash.py:6-33).

    positions [tokens, 3] (time, h, w), tags [tokens] (0 = video). keep: the
    kept row numbers in increasing order; inverse [tokens]: for a kept row
    its place in keep, for a dropped video row the place of its nearest kept
    video row of the same time (fp32 coordinates, first one on ties).
    """
    if positions.ndim != 2 or tags.ndim != 1 or positions.shape != (tags.numel(), 3):
        raise ValueError("Flash requires a single shared packed layout")
    video = tags == VIDEO_TAG
    if not bool(video.any()):
        raise ValueError("Flash requires video tokens")
    _lib.check_device(positions)
    on_grid = torch.ones_like(video)
    for axis in (1, 2):
        column = positions[:, axis]
        on_grid &= torch.isin(column, _retained(column[video], stride))
    kept = ~video | on_grid
    keep = kept.nonzero().flatten()
    inverse = torch.empty(tags.shape, dtype=torch.long, device=positions.device)
    inverse[keep] = torch.arange(keep.numel(), device=positions.device)
    dropped = (video & ~kept).nonzero().flatten()
    anchors = (video & kept).nonzero().flatten()
    if dropped.numel():
        coords = positions.to(torch.float32).contiguous()
        _lib.call("lr_flash_nearest_anchor", coords.data_ptr(), coords.shape[0], dropped.data_ptr(),
                  dropped.numel(), anchors.data_ptr(), anchors.numel(), inverse.data_ptr(),
                  _lib.stream(positions))
    return keep, inverse


def _check_config(blocks, config):
    compression = config["token_compression"]
    if len(blocks) != config["num_layers"]:
        raise ValueError("Flash depth and exported weights disagree")
    if (compression["reduction"] != "select" or compression["spatial_stride"] != 2
            or not compression["preserve_text_tokens"] or not compression["preserve_audio_tokens"]
            or compression.get("full_refresh_blocks")
            or compression.get("text_stride", 1) != 1 or compression.get("audio_stride", 1) != 1):
        raise ValueError("unsupported Flash token layout")
    start, end = compression["full_prefix_blocks"], len(blocks) - compression["full_suffix_blocks"]
    if not 0 < start < end < len(blocks):
        raise ValueError("Flash requires nonempty full-resolution prefix and suffix")
    return compression, start, end


def configure_flash(transformer, config):
    """Install Flash's selection hooks on a transformer (model/flash.py:36-96).

    Blocks [start, end) run on the kept rows; block `end` receives the
    restored full sequence. The block pre-hook arguments are (hidden, temb,
    adaLN indices, rotary (cos, sin), attention mask), as in the reference;
    hidden/indices/rotary/mask are gathered on their token dimension (1, 0,
    -2, -1). The hooks keep one forward's state at a time.
    """
    blocks = transformer.transformer_blocks
    compression, start, end = _check_config(blocks, config)
    if hasattr(transformer, "_lynnreal_flash_hooks"):
        raise ValueError("Flash is already configured")
    transformer.h3_token_compression = None
    signature = inspect.signature(transformer.forward)
    gain = float(compression.get("residual_gain", 1.0))
    state: dict = {}
    cache: dict = {}

    def begin(module, args, kwargs):
        if module.training or torch.is_grad_enabled():
            raise ValueError("Flash hooks require frozen inference")
        if state:
            raise RuntimeError("Flash transformer does not support concurrent forwards")
        bound = signature.bind(*args, **kwargs).arguments
        positions, tags = bound["position_ids"], bound["token_tags"]
        if not cache or not (torch.equal(positions, cache["positions"]) and torch.equal(tags, cache["tags"])):
            keep, inverse = spatial_layout(positions, tags)
            cache.update(positions=positions.clone(), tags=tags.clone(), keep=keep, inverse=inverse)
        state["keep"], state["inverse"] = cache["keep"], cache["inverse"]

    def compress(module, args):
        hidden, temb, indices, rotary, mask = args
        keep = state["keep"]
        if "full" not in state:
            state["full"] = hidden
            hidden = gather_rows(hidden, keep, 1)
            state["input"] = hidden
        return (hidden, temb, gather_rows(indices, keep, 0),
                tuple(gather_rows(value, keep, -2) for value in rotary),
                None if mask is None else gather_rows(mask, keep, -1))

    def restore_hook(module, args):
        hidden = restore(state.pop("full"), args[0], state.pop("input"), state["inverse"], gain)
        return (hidden, *args[1:])

    def finish(*_):
        state.clear()

    handles = [transformer.register_forward_pre_hook(begin, with_kwargs=True)]
    handles += [block.register_forward_pre_hook(compress) for block in blocks[start:end]]
    handles += [blocks[end].register_forward_pre_hook(restore_hook),
                transformer.register_forward_hook(finish, always_call=True)]
    transformer._lynnreal_flash_hooks = handles
