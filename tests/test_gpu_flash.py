"""GPU parity of Flash token selection (model/flash.py:6-96) through the C ABI:
the layout (keep, inverse) equal to the oracle's, the row gather equal to
index_select, the fused restore bit-exact vs the oracle, and the installed
hooks reproducing the reference's compress/restore sequence on a toy model."""
import numpy as np
import pytest
import torch
from torch import nn

from helpers import bf16_randn, to_np
from lynnreal_omni_amd import flash
from oracle import reference as ref
from test_flash_selection import _config, grid_layout

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("layout", [
    dict(frames=6, height=32, width=64, text=317),               # C5: 12288 video + 317 text rows
    dict(frames=5, height=33, width=61, text=40, audio=9),
    dict(frames=3, height=20, width=30, text=12, text_first=False),
    dict(frames=2, height=24, width=40, scale=0.125, origin=7.0),
], ids=["c5", "odd", "text_last", "dyadic"])
def test_layout_matches_oracle(layout):
    pos, tags = grid_layout(**layout)
    keep, inverse = flash.spatial_layout(pos.cuda(), tags.cuda())
    want_keep, want_inverse = ref.flash_spatial_layout(pos.numpy(), tags.numpy())
    assert np.array_equal(keep.cpu().numpy(), want_keep)
    assert np.array_equal(inverse.cpu().numpy(), want_inverse)


def test_layout_on_shuffled_float_rows():
    """Rows in a random order and irregular float coordinates: the nearest
    kept row and the first-of-equals rule follow row numbers, not grid order."""
    g = torch.Generator().manual_seed(11)
    pos, tags = grid_layout(frames=4, height=18, width=26, text=9)
    pos[:, 1:] = pos[:, 1:] * 0.37 + 0.01 * torch.rand(pos.shape[0], 2, generator=g, dtype=torch.float64)
    perm = torch.randperm(pos.shape[0], generator=g)
    pos, tags = pos[perm], tags[perm]
    keep, inverse = flash.spatial_layout(pos.cuda(), tags.cuda())
    want_keep, want_inverse = ref.flash_spatial_layout(pos.numpy(), tags.numpy())
    assert np.array_equal(keep.cpu().numpy(), want_keep)
    assert np.array_equal(inverse.cpu().numpy(), want_inverse)


@pytest.mark.parametrize("shape,dim,dtype", [
    ((2, 137, 5120), 1, torch.bfloat16),     # hidden rows (16-byte path)
    ((137,), 0, torch.int64),                # adaLN indices (byte path)
    ((137, 128), -2, torch.float32),         # rotary cos/sin rows
    ((2, 1, 137), -1, torch.bool),           # attention mask columns
    ((3, 137, 7), 1, torch.bfloat16),        # odd width (byte path)
])
def test_gather_rows_equals_index_select(shape, dim, dtype):
    g = torch.Generator().manual_seed(5)
    src = (torch.randn(shape, generator=g) * 100).to(dtype)
    n = shape[dim]
    index = torch.cat([torch.randperm(n, generator=g)[: n // 3], torch.tensor([0, n - 1, 0])])
    out = flash.gather_rows(src.cuda(), index.cuda(), dim)
    want = src.index_select(dim, index)
    assert out.is_contiguous() and out.dtype == dtype
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("batch,rows,compressed,width,gain", [
    (1, 12605, 3389, 5120, 1.0), (2, 137, 40, 5120, 0.75), (2, 37, 11, 7, 1.25), (1, 64, 64, 8, 0.0),
])
def test_restore_bit_exact(batch, rows, compressed, width, gain):
    g = torch.Generator().manual_seed(rows + width)
    full = bf16_randn((batch, rows, width), g)
    cur = bf16_randn((batch, compressed, width), g)
    inp = (cur.float() + 0.05 * torch.randn(batch, compressed, width, generator=g)).bfloat16()
    inverse = torch.randint(0, compressed, (rows,), generator=g)
    out = flash.restore(full.cuda(), cur.cuda(), inp.cuda(), inverse.cuda(), gain)
    want = ref.flash_restore(to_np(full), to_np(cur), to_np(inp), inverse.numpy(), gain)
    assert np.array_equal(to_np(out.cpu()), want)


class _Block(nn.Module):
    """Token-wise update that reads every gathered argument."""

    def __init__(self, i):
        super().__init__()
        self.i = i

    def forward(self, hidden, temb, indices, rotary, mask):
        cos, sin = rotary
        upd = hidden * 0.5 + (cos[:, :1] - sin[:, 1:2]).to(hidden.dtype)[None] + temb
        upd = upd + (indices.to(hidden.dtype) * 0.125)[None, :, None] * (self.i + 1)
        if mask is not None:
            upd = upd * mask[..., None].to(hidden.dtype)
        return upd


class _Transformer(nn.Module):
    def __init__(self, n):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([_Block(i) for i in range(n)])

    def forward(self, hidden_states, temb, adaln_indices, rotary_emb, position_ids, token_tags,
                attention_mask=None):
        for block in self.transformer_blocks:
            hidden_states = block(hidden_states, temb, adaln_indices, rotary_emb, attention_mask)
        return hidden_states


@torch.inference_mode()
def test_hooks_reproduce_compress_and_restore():
    pos, tags = grid_layout(frames=3, height=10, width=14, text=11)
    n = tags.numel()
    g = torch.Generator().manual_seed(9)
    x = bf16_randn((1, n, 64), g).cuda()
    temb = bf16_randn((1, 1, 64), g).cuda()
    indices = torch.randint(0, 6, (n,), generator=g).cuda()
    phase = torch.randn(n, 8, generator=g).cuda()
    rotary = (phase.cos(), phase.sin())
    mask = (torch.rand(1, n, generator=g) > 0.1).cuda()
    model = _Transformer(8).eval()
    config = _config(residual_gain=0.8)
    flash.configure_flash(model, config)
    got = model(x, temb, indices, rotary, pos.cuda(), tags.cuda(), mask)
    got2 = model(x, temb, indices, rotary, pos.cuda(), tags.cuda(), mask)   # cached layout
    assert torch.equal(got, got2)

    keep, inverse = (torch.from_numpy(a).cuda() for a in ref.flash_spatial_layout(pos.numpy(), tags.numpy()))
    blocks = _Transformer(8).eval().transformer_blocks      # the same blocks without hooks
    h = x
    for b in blocks[:2]:
        h = b(h, temb, indices, rotary, mask)
    full, small = h, h.index_select(1, keep)
    sub = (indices.index_select(0, keep), tuple(v.index_select(-2, keep) for v in rotary),
           mask.index_select(-1, keep))
    cur = small
    for b in blocks[2:6]:
        cur = b(cur, temb, sub[0], sub[1], sub[2])
    h = full + ((cur - small) * 0.8).index_select(1, inverse)
    for b in blocks[6:]:
        h = b(h, temb, indices, rotary, mask)
    assert torch.equal(got, h)


def _first_nearest(pos, dropped, anchors):
    """Brute force over anchors in increasing order: the first anchor of the
    row's time with the smallest squared (h, w) distance in fp64, else 0."""
    out = []
    for d in dropped:
        best, best_a = np.inf, 0
        for i, a in enumerate(anchors):
            if pos[a, 0] != pos[d, 0]:
                continue
            dist = (float(pos[d, 1]) - float(pos[a, 1])) ** 2 + (float(pos[d, 2]) - float(pos[a, 2])) ** 2
            if dist < best:
                best, best_a = dist, i
        out.append(best_a)
    return np.array(out)


def test_nearest_anchor_entry_point_ties_tiles_and_lonely_rows():
    """lr_flash_nearest_anchor directly: 3000 anchors (three LDS tiles, the
    nearest one in any lane's share), integer coordinates with many exact ties
    (the first anchor wins), and dropped rows of a time with no anchor (they
    take anchor 0)."""
    from lynnreal_omni_amd import _lib
    g = torch.Generator().manual_seed(21)
    tokens = 4200
    pos = torch.zeros(tokens, 3, dtype=torch.float32)
    pos[:, 0] = torch.randint(0, 4, (tokens,), generator=g).float()
    pos[:, 1:] = torch.randint(0, 40, (tokens, 2), generator=g).float()
    order = torch.randperm(tokens, generator=g)
    anchors = order[:3000].sort().values
    dropped = order[3000:].sort().values
    pos[dropped[:50], 0] = 9.0  # a time with no anchor
    inverse = torch.arange(tokens, dtype=torch.int64) * 7 + 3
    pos_d, anchors_d, dropped_d, inverse_d = pos.cuda(), anchors.cuda(), dropped.cuda(), inverse.cuda()
    _lib.call("lr_flash_nearest_anchor", pos_d.data_ptr(), tokens, dropped_d.data_ptr(), dropped.numel(),
              anchors_d.data_ptr(), anchors.numel(), inverse_d.data_ptr(), _lib.stream(pos_d))
    torch.cuda.synchronize()
    pick = _first_nearest(pos.numpy(), dropped.numpy(), anchors.numpy())
    want = inverse.numpy().copy()
    want[dropped.numpy()] = inverse.numpy()[anchors.numpy()[pick]]
    assert (pick[:50] == 0).all()
    assert np.array_equal(inverse_d.cpu().numpy(), want)
