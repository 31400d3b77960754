"""The C3 projection chain at its full size on gfx950 (benchmark config 3: T=12288,
D=5120, FFN 20480 with GELU-tanh; model/fusion.py:61-98 with the FFN-down gated
residual in the GEMM epilogue), checked through row independence: every op of
the chain (norm + modulate + quantize, the projections, the re-quantizations,
the gated residuals) is row-wise, so each output row must equal the oracle's
chain run on that row alone. QKV and the first residual are compared bit for
bit; the block output follows the GELU (hardware exp2 / reciprocal) and is
compared within the bf16 tolerance (max relative error 1e-2, cosine 0.9999)."""
import types

import numpy as np
import pytest
import torch

from helpers import bf16_randn, to_np
from lynnreal_omni_amd import fusion
from lynnreal_omni_amd.int8 import Int8Linear
from oracle import bf16
from oracle import reference as ref

pytestmark = pytest.mark.gpu

T, D, F = 12288, 5120, 20480
# first and last rows, both sides of 256-row tile edges, and rows inside tiles
ROWS = [0, 1, 255, 256, 4097, 8191, 8192, 12030, 12287]


def _weights(g, n, k):
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
    s = torch.rand(n, 1, generator=g) * 4e-3 + 1e-3
    b = (0.02 * torch.randn(n, generator=g)).bfloat16()
    return w, s, b


@torch.inference_mode()
def test_c3_chain_full_size_rows_match_oracle():
    g = torch.Generator().manual_seed(20261201 + 2)
    x = bf16_randn((1, T, D), g, outliers=0.01)
    attn = bf16_randn((1, T, D), g)
    table = (0.1 * torch.randn(1, 6 * D, generator=g)).bfloat16()
    idx = torch.zeros(T, dtype=torch.int64)
    gamma = (1 + 0.05 * torch.randn(D, generator=g)).bfloat16()
    packed = {"to_qkv": _weights(g, 3 * D, D), "to_out": _weights(g, D, D),
              "up": _weights(g, F, D), "down": _weights(g, D, F)}
    dev = torch.device("cuda")
    layers = fusion.ChainLayers(**{name: Int8Linear.from_packed(w.to(dev), s.to(dev), b.to(dev), gemm="hip")
                                   for name, (w, s, b) in packed.items()})
    norm = types.SimpleNamespace(weight=gamma.to(dev), eps=1e-6)
    qkv, x1, x2 = fusion.projection_chain(x.to(dev), layers, norm, norm, table.to(dev), idx.to(dev),
                                          attn.to(dev))
    sel = torch.tensor(ROWS, device=dev)
    got_qkv, got_x1, got_x2 = (to_np(v.reshape(T, -1).index_select(0, sel)) for v in (qkv, x1, x2))

    r = len(ROWS)
    X = to_np(x[0, ROWS]).reshape(1, r, D)
    A = to_np(attn[0, ROWS])
    Tb, G, I = to_np(table), to_np(gamma), idx[ROWS].numpy()
    W = {k: (v[0].numpy(), v[1].numpy().reshape(-1), to_np(v[2])) for k, v in packed.items()}
    q1, s1 = ref.rms_adaln_quant(X, G, Tb, I, 0, 1, 1e-6)
    want_qkv = ref.dequant(ref.int_mm(q1, W["to_qkv"][0]), s1, W["to_qkv"][1], W["to_qkv"][2])
    assert np.array_equal(got_qkv, want_qkv), "QKV rows"
    qa, sa = ref.quantize_rows(A)
    o = ref.dequant(ref.int_mm(qa, W["to_out"][0]), sa, W["to_out"][1], W["to_out"][2])
    X1 = ref.gated_residual(X, o.reshape(1, r, D), Tb, I, 2)
    assert np.array_equal(got_x1, X1.reshape(r, D)), "residual after the out-projection"
    q2, s2 = ref.rms_adaln_quant(X1, G, Tb, I, 3, 4, 1e-6)
    h = ref.gelu_tanh(ref.dequant(ref.int_mm(q2, W["up"][0]), s2, W["up"][1], W["up"][2]))
    q3, s3 = ref.quantize_rows(h)
    dn = ref.dequant(ref.int_mm(q3, W["down"][0]), s3, W["down"][1], W["down"][2])
    X2 = ref.gated_residual(X1, dn.reshape(1, r, D), Tb, I, 5).reshape(r, D)

    a = bf16.to_f32(got_x2).astype(np.float64)
    e = bf16.to_f32(X2).astype(np.float64)
    for row in range(r):
        cos = float(a[row] @ e[row] / (np.linalg.norm(a[row]) * np.linalg.norm(e[row])))
        assert cos >= 0.9999, (ROWS[row], cos)
        big = np.abs(e[row]) > 1e-3 * np.abs(e[row]).max()
        rel = np.abs(a[row][big] - e[row][big]) / np.abs(e[row][big])
        assert rel.max() <= 1e-2, (ROWS[row], rel.max())
