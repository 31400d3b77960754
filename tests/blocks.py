"""A small DiT block with the submodule layout the fused block expects
(MiniMax H3's: norm1/norm2 with weight and eps, attn.to_qkv/to_out/norm_q/
norm_k/heads/processor, ff.net[0].proj and ff.net[2], adaln_proj.linear and
.hidden_size), for tests that install the fused block surface. diffusers is
not installed here, so its block class cannot be used."""
import torch
from torch import nn

from lynnreal_omni_amd.int8 import Int8Linear


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        x32 = x.float()
        y = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class NativeProcessor:
    _attention_backend = "native"
    _parallel_config = None

    def __call__(self, attn, hidden_states, rotary_emb=None, attention_mask=None):
        return attn.to_out[0](hidden_states)


class Attention(nn.Module):
    def __init__(self, dim, heads, layers):
        super().__init__()
        self.heads = heads
        self.to_qkv = layers["qkv"]
        self.to_out = nn.ModuleList([layers["out"], nn.Dropout(0.0)])
        self.norm_q = RMSNorm(dim // heads)
        self.norm_k = RMSNorm(dim // heads)
        self.fused_projections = True
        self.processor = NativeProcessor()

    def set_processor(self, processor):
        self.processor = processor

    def forward(self, hidden_states, rotary_emb=None, attention_mask=None):
        return self.processor(self, hidden_states, rotary_emb, attention_mask)


class _Proj(nn.Module):
    def __init__(self, layer):
        super().__init__()
        self.proj = layer


class FeedForward(nn.Module):
    def __init__(self, layers):
        super().__init__()
        self.net = nn.ModuleList([_Proj(layers["up"]), nn.Dropout(0.0), layers["down"]])


class AdaLNProj(nn.Module):
    def __init__(self, time_dim, dim):
        super().__init__()
        self.linear = nn.Linear(time_dim, 6 * dim)
        self.hidden_size = dim


class Block(nn.Module):
    """forward() is a plain stand-in (the native path a guarded block falls back to)."""

    def __init__(self, dim, heads, inner, time_dim, gen):
        super().__init__()
        layers = {}
        for name, n, k in (("qkv", 3 * dim, dim), ("out", dim, dim), ("up", 2 * inner, dim),
                           ("down", dim, inner)):
            w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=gen)
            s = torch.rand(n, 1, generator=gen) * 4e-3 + 1e-3
            b = (0.02 * torch.randn(n, generator=gen)).bfloat16()
            layers[name] = Int8Linear.from_packed(w, s, b, "triton")
        self.norm1, self.norm2 = RMSNorm(dim), RMSNorm(dim)
        with torch.no_grad():
            for norm in (self.norm1, self.norm2):
                norm.weight.copy_(1 + 0.05 * torch.randn(dim, generator=gen))
        self.attn = Attention(dim, heads, layers)
        self.ff = FeedForward(layers)
        self.adaln_proj = AdaLNProj(time_dim, dim)
        with torch.no_grad():
            self.adaln_proj.linear.weight.copy_(0.02 * torch.randn(6 * dim, time_dim, generator=gen))
            self.adaln_proj.linear.bias.copy_(0.1 * torch.randn(6 * dim, generator=gen))

    def forward(self, hidden_states, temb, adaln_indices, rotary_emb, attention_mask=None):
        return hidden_states + 0 * temb.sum()


class Transformer(nn.Module):
    def __init__(self, blocks):
        super().__init__()
        self.transformer_blocks = nn.ModuleList(blocks)

    def forward(self, hidden_states, temb, adaln_indices, rotary_emb, timestep=None):
        for block in self.transformer_blocks:
            hidden_states = block(hidden_states, temb, adaln_indices, rotary_emb)
        return hidden_states
