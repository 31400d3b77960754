"""Flash token selection (model/flash.py:6-96): the oracle and the host logic (CPU).

The reference ships no fixtures for it; the oracle's layout is pinned by
torch's own unique/isin/cdist/argmin (oracle/torch_path.py) on integer and
dyadic grids, where the fp32 distance is exact and both must agree row for
row, by the closed form of a full stride-2 grid, and by brute force (every
dropped row lands on a kept row of its time at the least distance). The
restore is pinned by torch's bf16 CPU arithmetic of the reference's own
expression. configure_flash's validation runs before any kernel.
"""
import numpy as np
import pytest
import torch
from torch import nn

from helpers import bf16_randn, to_np
from lynnreal_omni_amd import flash
from oracle import reference as ref, torch_path as tp


def grid_layout(frames, height, width, text=0, audio=0, scale=1.0, origin=0.0, text_first=True):
    """Packed positions (time, h, w) and tags: text rows (tag 1), video rows
    (tag 0) in (time, h, w) order, audio rows (tag 2)."""
    rows, tags = [], []
    text_rows = [[float(i), 0.0, 0.0] for i in range(text)]
    video = [[origin + t, scale * h, scale * w] for t in range(frames) for h in range(height)
             for w in range(width)]
    audio_rows = [[origin + i, 0.0, 0.0] for i in range(audio)]
    if text_first:
        rows, tags = text_rows + video, [1] * text + [0] * len(video)
    else:
        rows, tags = video + text_rows, [0] * len(video) + [1] * text
    rows += audio_rows
    tags += [2] * audio
    return torch.tensor(rows, dtype=torch.float64), torch.tensor(tags)


LAYOUTS = [
    dict(frames=1, height=4, width=4),                          # direct cdist path (<= 25 rows)
    dict(frames=3, height=5, width=7, text=4),
    dict(frames=2, height=8, width=6, text=3, audio=5),
    dict(frames=6, height=16, width=32, text=17),               # mm cdist path
    dict(frames=4, height=9, width=11, text=7, text_first=False),
    dict(frames=2, height=12, width=10, scale=0.25, origin=3.0),  # dyadic, exact in fp32
]


@pytest.mark.parametrize("layout", LAYOUTS, ids=lambda d: "x".join(str(v) for v in d.values()))
def test_layout_matches_torch_cdist(layout):
    pos, tags = grid_layout(**layout)
    keep, inverse = ref.flash_spatial_layout(pos.numpy(), tags.numpy())
    tkeep, tinverse = tp.flash_spatial_layout(pos, tags)
    assert np.array_equal(keep, tkeep.numpy())
    assert np.array_equal(inverse, tinverse.numpy())


@pytest.mark.parametrize("frames,height,width", [(2, 6, 8), (3, 7, 9), (1, 5, 4)])
def test_layout_closed_form_full_grid(frames, height, width):
    """Stride 2 keeps h in {0, 2, ...} + {H-1} (likewise w). A dropped row is
    one step from a kept row on each dropped axis; of the equidistant kept
    rows the first in (time, h, w) order wins: (h-1, w-1) and so on."""
    text = 3
    pos, tags = grid_layout(frames, height, width, text=text)
    keep, inverse = ref.flash_spatial_layout(pos.numpy(), tags.numpy())
    kept_h = set(range(0, height, 2)) | {height - 1}
    kept_w = set(range(0, width, 2)) | {width - 1}

    def row(t, h, w):
        return text + (t * height + h) * width + w

    want_keep = list(range(text)) + [row(t, h, w) for t in range(frames) for h in range(height)
                                     for w in range(width) if h in kept_h and w in kept_w]
    assert keep.tolist() == want_keep
    place = {r: i for i, r in enumerate(want_keep)}
    for t in range(frames):
        for h in range(height):
            for w in range(width):
                ah = h if h in kept_h else h - 1
                aw = w if w in kept_w else w - 1
                assert inverse[row(t, h, w)] == place[row(t, ah, aw)]
    assert inverse[:text].tolist() == list(range(text))


def test_layout_brute_force_on_irregular_float_grid():
    """Non-uniform float coordinates (no ties): every dropped row maps to a
    kept video row of its own time at the least fp32-coordinate distance,
    and torch's cdist picks the same row wherever its fp32 rounding leaves
    the order intact (the two nearest differ by more than 1e-3)."""
    g = torch.Generator().manual_seed(3)
    frames, height, width = 3, 9, 10
    hs = torch.cumsum(torch.rand(height, generator=g, dtype=torch.float64) + 0.3, 0)
    ws = torch.cumsum(torch.rand(width, generator=g, dtype=torch.float64) + 0.3, 0)
    rows = [[0.5 * t, hs[h], ws[w]] for t in range(frames) for h in range(height) for w in range(width)]
    pos = torch.tensor(rows, dtype=torch.float64)
    tags = torch.zeros(len(rows), dtype=torch.long)
    keep, inverse = ref.flash_spatial_layout(pos.numpy(), tags.numpy())
    tkeep, tinverse = tp.flash_spatial_layout(pos, tags)
    assert np.array_equal(keep, tkeep.numpy())
    p = pos.numpy().astype(np.float32).astype(np.float64)
    kept = set(keep.tolist())
    agree = 0
    for r in range(len(rows)):
        if r in kept:
            assert keep[inverse[r]] == r
            continue
        same_time = [a for a in keep if p[a, 0] == p[r, 0]]
        d = {a: (p[r, 1] - p[a, 1]) ** 2 + (p[r, 2] - p[a, 2]) ** 2 for a in same_time}
        best = min(d.values())
        assert d[keep[inverse[r]]] == best
        second = min([v for a, v in d.items() if v > best], default=np.inf)
        if second - best > 1e-3:
            assert tinverse[r] == inverse[r]
            agree += 1
    assert agree > 0


def test_layout_row_without_same_time_anchor_takes_first():
    # A lone video row at a time with no kept row: argmin over +inf -> the first anchor.
    pos = torch.tensor([[0, 0, 0], [0, 0, 2], [0, 0, 1], [5, 0, 1]], dtype=torch.float64)
    tags = torch.zeros(4, dtype=torch.long)
    keep, inverse = ref.flash_spatial_layout(pos.numpy(), tags.numpy())
    tkeep, tinverse = tp.flash_spatial_layout(pos, tags)
    assert keep.tolist() == [0, 1] and inverse.tolist() == [0, 1, 0, 0]
    assert np.array_equal(inverse, tinverse.numpy())


@pytest.mark.parametrize("gain", [1.0, 0.5, 1.25, 0.0, -0.3])
def test_restore_matches_torch_bf16(gain):
    g = torch.Generator().manual_seed(4)
    full = bf16_randn((2, 37, 24), g)
    cur = bf16_randn((2, 11, 24), g)
    inp = (cur.float() + 0.01 * torch.randn(2, 11, 24, generator=g)).bfloat16()
    inverse = torch.randint(0, 11, (37,), generator=g)
    ours = ref.flash_restore(to_np(full), to_np(cur), to_np(inp), inverse.numpy(), gain)
    theirs = tp.flash_restore(full, cur, inp, inverse, gain)
    assert np.array_equal(ours, to_np(theirs))


def test_restore_rounds_each_step():
    # cur - inp = 1 + 2^-7 - 2^-8 = 1 + 2^-8 is a bf16 tie and rounds to 1
    # before it meets full = -1: the result is 0, not the unrounded 2^-8.
    full = torch.tensor([[[-1.0]]]).bfloat16()
    cur = torch.tensor([[[1.0 + 2.0 ** -7]]]).bfloat16()
    inp = torch.tensor([[[2.0 ** -8]]]).bfloat16()
    out = ref.flash_restore(to_np(full), to_np(cur), to_np(inp), np.array([0]), 1.0)
    assert out.tolist() == [[[0]]]
    assert to_np(tp.flash_restore(full, cur, inp, torch.tensor([0]), 1.0)).tolist() == out.tolist()


def test_spatial_layout_rejects_bad_layouts():
    with pytest.raises(ValueError, match="single shared packed layout"):
        flash.spatial_layout(torch.zeros(4, 2), torch.zeros(4, dtype=torch.long))
    with pytest.raises(ValueError, match="single shared packed layout"):
        flash.spatial_layout(torch.zeros(4, 3), torch.zeros(5, dtype=torch.long))
    with pytest.raises(ValueError, match="requires video tokens"):
        flash.spatial_layout(torch.zeros(4, 3), torch.ones(4, dtype=torch.long))
    with pytest.raises(ValueError, match="GPU tensors"):
        flash.spatial_layout(torch.zeros(4, 3), torch.zeros(4, dtype=torch.long))


class _Block(nn.Module):
    def forward(self, hidden, temb, indices, rotary, mask):
        return hidden


class _Transformer(nn.Module):
    def __init__(self, n):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([_Block() for _ in range(n)])

    def forward(self, hidden_states, temb, adaln_indices, rotary_emb, position_ids, token_tags,
                attention_mask=None):
        for block in self.transformer_blocks:
            hidden_states = block(hidden_states, temb, adaln_indices, rotary_emb, attention_mask)
        return hidden_states


def _config(**kw):
    compression = {"reduction": "select", "spatial_stride": 2, "preserve_text_tokens": True,
                   "preserve_audio_tokens": True, "full_prefix_blocks": 2, "full_suffix_blocks": 2}
    compression.update(kw)
    return {"num_layers": 8, "token_compression": compression}


@pytest.mark.parametrize("change,match", [
    ({"reduction": "mean"}, "unsupported Flash token layout"),
    ({"spatial_stride": 4}, "unsupported Flash token layout"),
    ({"preserve_text_tokens": False}, "unsupported Flash token layout"),
    ({"full_refresh_blocks": [4]}, "unsupported Flash token layout"),
    ({"text_stride": 2}, "unsupported Flash token layout"),
    ({"full_prefix_blocks": 0}, "nonempty full-resolution prefix and suffix"),
    ({"full_suffix_blocks": 0}, "nonempty full-resolution prefix and suffix"),
    ({"full_prefix_blocks": 4, "full_suffix_blocks": 4}, "nonempty full-resolution prefix and suffix"),
])
def test_configure_flash_rejects_unsupported_configs(change, match):
    with pytest.raises(ValueError, match=match):
        flash.configure_flash(_Transformer(8), _config(**change))


def test_configure_flash_checks_depth_and_installs_once():
    with pytest.raises(ValueError, match="depth and exported weights disagree"):
        flash.configure_flash(_Transformer(7), _config())
    model = _Transformer(8)
    flash.configure_flash(model, _config())
    assert model.h3_token_compression is None and len(model._lynnreal_flash_hooks) == 1 + 4 + 1 + 1
    with pytest.raises(ValueError, match="already configured"):
        flash.configure_flash(model, _config())


def test_flash_hooks_require_frozen_inference():
    model = _Transformer(8).eval()
    flash.configure_flash(model, _config())
    pos, tags = grid_layout(1, 4, 4)
    x = torch.zeros(1, tags.numel(), 8)
    with pytest.raises(ValueError, match="frozen inference"):
        model(x, None, torch.zeros(tags.numel(), dtype=torch.long), (x[0], x[0]), pos, tags)
