"""bf16 DiT block with only the element-wise fusions (drop-in for the
reference's model/elementwise_fusion.py).

The block keeps its own normalisation, attention and projections; the adaLN
table comes from kernels.adaln_table, the two residual updates become
_gated_residual and the FFN activation _swiglu, all gfx950 kernels. Blocks
are duck-typed like the reference's H3 block: `adaln_proj.linear`,
`adaln_proj.hidden_size`, `norm1`, `norm2`, `attn`, `ff.net[0].proj`,
`ff.net[2]`.
"""
from __future__ import annotations

from types import MethodType

from .kernels import _gated_residual, _swiglu, adaln_table


def _modulation_table(block, temb):
    """linear(F.silu(temb).to(bf16)).view(-1, 6 * hidden) (model/elementwise_fusion.py:8-10)."""
    linear = block.adaln_proj.linear
    return adaln_table(temb, linear.weight, linear.bias).view(-1, 6 * block.adaln_proj.hidden_size)


def _modulate(normalized, table, indices, shift_slot, scale_slot, width):
    shift = table[:, shift_slot * width:(shift_slot + 1) * width].index_select(0, indices)
    scale = table[:, scale_slot * width:(scale_slot + 1) * width].index_select(0, indices)
    return normalized * (1 + scale) + shift


def block_forward(self, hidden_states, temb, adaln_indices, rotary_emb, attention_mask=None):
    """One block: attention and FFN with fused gated residuals and SwiGLU
    (model/elementwise_fusion.py:7-20)."""
    width = self.adaln_proj.hidden_size
    table = _modulation_table(self, temb)
    attn_in = _modulate(self.norm1(hidden_states), table, adaln_indices, 0, 1, width)
    update = self.attn(attn_in, rotary_emb, attention_mask)
    hidden_states = _gated_residual(hidden_states, update, table, adaln_indices, 2)
    ffn_in = _modulate(self.norm2(hidden_states), table, adaln_indices, 3, 4, width)
    update = self.ff.net[2](_swiglu(self.ff.net[0].proj(ffn_in)))
    return _gated_residual(hidden_states, update, table, adaln_indices, 5)


def enable_elementwise_fusion(transformer, fused_quant=False):
    """Patch every block's forward (model/elementwise_fusion.py:23-30)."""
    if fused_quant or transformer.training:
        raise ValueError("elementwise fusion requires an evaluation-mode BF16 model")
    blocks = transformer.transformer_blocks
    for block in blocks:
        block.forward = MethodType(block_forward, block)
    return {"kind": "elementwise", "swiglu": True, "gated_residual": True,
            "normalization": "native", "attention_processor": "native",
            "blocks": len(blocks), "activation_quantization_fused": False}
