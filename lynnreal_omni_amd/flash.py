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
    _lib.same_device(full, current=current, input=input)
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


def _on_grid(coordinate: torch.Tensor, alphabet: torch.Tensor, stride: int) -> torch.Tensor:
    """Whether each coordinate (a member of the sorted `alphabet` of distinct
    values) is every stride-th distinct value counting from the smallest, or
    the largest one: its rank in the alphabet decides."""
    rank = torch.searchsorted(alphabet, coordinate.contiguous())
    return (rank % stride == 0) | (rank == alphabet.numel() - 1)


def spatial_layout(positions: torch.Tensor, tags: torch.Tensor, stride: int = 2):
    """(keep, inverse) of the Flash selection (model/flash.py:6-33).

    positions [tokens, 3] (time, h, w), tags [tokens] (0 = video). A video row
    is kept when both its h and w are on the stride grid of the video rows'
    distinct values (the largest value always counts); every other row is
    kept. keep: the kept row numbers in increasing order. inverse [tokens]: a
    kept row's place in keep; a dropped row's is its nearest kept video row
    of the same time (fp32 coordinates, first one on ties), found by the
    nearest-anchor kernel.
    """
    if positions.ndim != 2 or tags.ndim != 1 or positions.shape != (tags.numel(), 3):
        raise ValueError("Flash requires a single shared packed layout")
    video = tags == VIDEO_TAG
    if not bool(video.any()):
        raise ValueError("Flash requires video tokens")
    _lib.check_device(positions)
    _lib.same_device(positions, tags=tags)
    grid = video.clone()
    rows = positions[video]
    for axis in (1, 2):
        grid[video] &= _on_grid(rows[:, axis], torch.unique(rows[:, axis], sorted=True), stride)
    kept = ~video | grid
    keep = kept.nonzero().flatten()
    # a kept row's place among the kept rows is the running count of kept rows before it
    inverse = torch.cumsum(kept, 0) - 1
    dropped = (~kept).nonzero().flatten()
    if dropped.numel():
        anchors = grid.nonzero().flatten()
        coords = positions.to(torch.float32).contiguous()
        _lib.call("lr_flash_nearest_anchor", coords.data_ptr(), coords.shape[0], dropped.data_ptr(),
                  dropped.numel(), anchors.data_ptr(), anchors.numel(), inverse.data_ptr(),
                  _lib.stream(positions))
    return keep, inverse


# The one token layout the trained Flash blocks support: spatial selection with
# stride 2, every text and audio row kept, no refresh blocks. Each entry is
# (key, value when absent or None to require the key, test).
_LAYOUT_RULES = (
    ("reduction", None, lambda v: v == "select"),
    ("spatial_stride", None, lambda v: v == 2),
    ("preserve_text_tokens", None, bool),
    ("preserve_audio_tokens", None, bool),
    ("full_refresh_blocks", False, lambda v: not v),
    ("text_stride", 1, lambda v: v == 1),
    ("audio_stride", 1, lambda v: v == 1),
)


def _compressed_span(blocks, config):
    """Blocks [start, end) that run on the kept rows, and the restore gain."""
    if len(blocks) != config["num_layers"]:
        raise ValueError("Flash depth and exported weights disagree")
    compression = config["token_compression"]
    for key, absent, test in _LAYOUT_RULES:
        value = compression[key] if absent is None else compression.get(key, absent)
        if not test(value):
            raise ValueError("unsupported Flash token layout")
    start = compression["full_prefix_blocks"]
    end = len(blocks) - compression["full_suffix_blocks"]
    if not 0 < start < end < len(blocks):
        raise ValueError("Flash requires nonempty full-resolution prefix and suffix")
    return start, end, float(compression.get("residual_gain", 1.0))


class _FlashForward:
    """Hook state of one Flash transformer: the layout of the current forward
    (cached across forwards with equal positions and tags) and, between the
    first compressed block and the restore, the full-resolution hidden rows
    and the compressed rows that entered the compressed span."""

    def __init__(self, transformer, gain):
        self.signature = inspect.signature(transformer.forward)
        self.gain = gain
        self.layout = None          # (positions, tags, keep, inverse) of the last layout built
        self.current = None         # (keep, inverse) while a forward runs
        self.full = self.entered = None

    def begin(self, module, args, kwargs):
        if module.training or torch.is_grad_enabled():
            raise ValueError("Flash hooks require frozen inference")
        if self.current is not None:
            raise RuntimeError("Flash transformer does not support concurrent forwards")
        bound = self.signature.bind(*args, **kwargs).arguments
        positions, tags = bound["position_ids"], bound["token_tags"]
        cached = self.layout
        if cached is None or not (torch.equal(positions, cached[0]) and torch.equal(tags, cached[1])):
            cached = self.layout = (positions.clone(), tags.clone(), *spatial_layout(positions, tags))
        self.current = cached[2:]

    def compress(self, module, args):
        hidden, temb, indices, rotary, mask = args
        keep = self.current[0]
        if self.full is None:           # the first compressed block: drop rows once
            self.full, hidden = hidden, gather_rows(hidden, keep, 1)
            self.entered = hidden
        return (hidden, temb, gather_rows(indices, keep, 0),
                tuple(gather_rows(value, keep, -2) for value in rotary),
                None if mask is None else gather_rows(mask, keep, -1))

    def restore(self, module, args):
        hidden = restore(self.full, args[0], self.entered, self.current[1], self.gain)
        self.full = self.entered = None
        return (hidden, *args[1:])

    def finish(self, *_):
        self.current = self.full = self.entered = None


def configure_flash(transformer, config):
    """Install Flash's selection hooks on a transformer (model/flash.py:36-96).

    Blocks [start, end) run on the kept rows; block `end` receives the
    restored full sequence. The block pre-hook arguments are (hidden, temb,
    adaLN indices, rotary (cos, sin), attention mask), as in the reference;
    hidden/indices/rotary/mask are gathered on their token dimension (1, 0,
    -2, -1). One forward runs at a time.
    """
    blocks = transformer.transformer_blocks
    start, end, gain = _compressed_span(blocks, config)
    if hasattr(transformer, "_lynnreal_flash_hooks"):
        raise ValueError("Flash is already configured")
    transformer.h3_token_compression = None
    run = _FlashForward(transformer, gain)
    handles = [transformer.register_forward_pre_hook(run.begin, with_kwargs=True)]
    handles += [block.register_forward_pre_hook(run.compress) for block in blocks[start:end]]
    handles += [blocks[end].register_forward_pre_hook(run.restore),
                transformer.register_forward_hook(run.finish, always_call=True)]
    transformer._lynnreal_flash_hooks = handles
