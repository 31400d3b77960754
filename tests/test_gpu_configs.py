"""GPU parity at the benchmark configs' own shapes.

C1 and the M=256 projections are compared over their whole outputs with the
oracle's torch restatement (oracle/torch_path.py, which tests/test_oracle.py
pins bit for bit against the C oracle): int8 activations, row scales and the
bf16 GEMM outputs must be identical. The ragged C5 chain (T = 12288 video +
317 text tokens, six per-frame modulation rows) and the reference FFN
(SwiGLU, model/kernels.py:169-185) at full size are row-wise, so sampled rows
(tile edges, frame boundaries, the text tail) must equal the C oracle's chain
run on those rows alone. Everything before the FFN activation is compared bit
for bit; what follows GELU or the sigmoid (hardware exp2 / reciprocal) within
the bf16 tolerance (max relative error 1e-2, cosine 0.9999).
"""
import types

import numpy as np
import pytest
import torch

from helpers import bf16_randn, to_np
from lynnreal_omni_amd import fusion, kernels
from lynnreal_omni_amd.int8 import Int8Linear
from lynnreal_omni_amd.int8_gemm import int8_matmul, int8_matmul_int32
from oracle import bf16
from oracle import reference as ref
from oracle import torch_path as tp

pytestmark = pytest.mark.gpu

D = 5120


def _weights(g, n, k):
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
    s = torch.rand(n, 1, generator=g) * 4e-3 + 1e-3
    b = (0.02 * torch.randn(n, generator=g)).bfloat16()
    return w, s, b


def _assert_rows_close(got_u16, want_u16, rows):
    a = bf16.to_f32(got_u16).astype(np.float64)
    e = bf16.to_f32(want_u16).astype(np.float64)
    for i, row in enumerate(rows):
        cos = float(a[i] @ e[i] / (np.linalg.norm(a[i]) * np.linalg.norm(e[i])))
        assert cos >= 0.9999, (row, cos)
        big = np.abs(e[i]) > 1e-3 * np.abs(e[i]).max()
        rel = np.abs(a[i][big] - e[i][big]) / np.abs(e[i][big])
        assert rel.max() <= 1e-2, (row, rel.max())


@torch.inference_mode()
def test_c1_linear_whole_output_bit_exact():
    """X bf16 [2048, 5120] with 1% outlier channels x20 ->
    quantize_rows -> INT8 GEMM (N = 5120, auto tile) + bias -> bf16."""
    g = torch.Generator().manual_seed(20261201 + 0)
    m, k, n = 2048, 5120, 5120
    x = bf16_randn((m, k), g, outliers=0.01)
    w, s, b = _weights(g, n, k)
    q, qs = kernels.quantize_rows(x.cuda())
    y = int8_matmul(q, w.cuda().t(), qs, s.cuda(), b.cuda())
    want_q, want_s = tp.quantize(x)
    assert torch.equal(q.cpu(), want_q) and torch.equal(qs.cpu(), want_s)
    want = tp.epilogue(tp.int_mm(want_q, w), want_s, s.reshape(1, -1), b)
    assert torch.equal(y.cpu(), want)


@torch.inference_mode()
@pytest.mark.parametrize("tile", [None, (128, 160), (64, 80), (256, 80)], ids=str)
@pytest.mark.parametrize("n", [5120, 20480])
@pytest.mark.parametrize("m", [256, 200, 64, 1])
def test_skinny_projection_whole_output_bit_exact(m, n, tile):
    """BASELINE config 5's decode-like projections (M = 256, K = 5120, N = 5120
    and 20480) and smaller M, through the auto tile and each small-M tile:
    int32 accumulators and the bf16 epilogue over the whole output."""
    q, qs, w, s, b, want_acc, want_y = _skinny_case(m, n)
    wd = w.cuda()
    acc = int8_matmul_int32(q.cuda(), wd.t(), tile=tile)
    assert torch.equal(acc.cpu(), want_acc)
    y = int8_matmul(q.cuda(), wd.t(), qs.cuda(), s.cuda(), b.cuda(), tile=tile)
    assert torch.equal(y.cpu(), want_y)


_SKINNY = {}


def _skinny_case(m, n):
    """Inputs and CPU-oracle outputs of one skinny shape, computed once per
    shape for all the tiles that are checked against them."""
    if (m, n) not in _SKINNY:
        g = torch.Generator().manual_seed(20261201 + 4 + m + n)
        k = 5120
        x = bf16_randn((m, k), g, outliers=0.01)
        w, s, b = _weights(g, n, k)
        q, qs = tp.quantize(x)
        want_acc = tp.int_mm(q, w)
        _SKINNY.clear()
        _SKINNY[(m, n)] = (q, qs, w, s, b, want_acc, tp.epilogue(want_acc, qs, s.reshape(1, -1), b))
    return _SKINNY[(m, n)]


def _c5_inputs(g, video=12288, text=317, ffn=20480, up=None):
    t = video + text
    x = bf16_randn((1, t, D), g, outliers=0.01)
    attn = bf16_randn((1, t, D), g)
    table = (0.1 * torch.randn(6, 6 * D, generator=g)).bfloat16()
    idx = torch.cat([torch.clamp(torch.arange(video) // 2048, max=5), torch.zeros(text, dtype=torch.int64)])
    gamma = (1 + 0.05 * torch.randn(D, generator=g)).bfloat16()
    packed = {"to_qkv": _weights(g, 3 * D, D), "to_out": _weights(g, D, D),
              "up": _weights(g, up or ffn, D), "down": _weights(g, D, ffn)}
    return t, x, attn, table, idx, gamma, packed


def _run_chain(x, attn, table, idx, gamma, packed, ffn):
    dev = torch.device("cuda")
    layers = fusion.ChainLayers(**{name: Int8Linear.from_packed(w.to(dev), s.to(dev), b.to(dev), gemm="hip")
                                   for name, (w, s, b) in packed.items()})
    norm = types.SimpleNamespace(weight=gamma.to(dev), eps=1e-6)
    return fusion.projection_chain(x.to(dev), layers, norm, norm, table.to(dev), idx.to(dev), attn.to(dev),
                                   ffn=ffn)


def _oracle_front(rows, x, attn, table, idx, gamma, packed):
    r = len(rows)
    X = to_np(x[0, rows]).reshape(1, r, D)
    A = to_np(attn[0, rows])
    Tb, G, I = to_np(table), to_np(gamma), idx[rows].numpy()
    W = {k: (v[0].numpy(), v[1].numpy().reshape(-1), to_np(v[2])) for k, v in packed.items()}
    q1, s1 = ref.rms_adaln_quant(X, G, Tb, I, 0, 1, 1e-6)
    qkv = ref.dequant(ref.int_mm(q1, W["to_qkv"][0]), s1, W["to_qkv"][1], W["to_qkv"][2])
    qa, sa = ref.quantize_rows(A)
    o = ref.dequant(ref.int_mm(qa, W["to_out"][0]), sa, W["to_out"][1], W["to_out"][2])
    X1 = ref.gated_residual(X, o.reshape(1, r, D), Tb, I, 2)
    q2, s2 = ref.rms_adaln_quant(X1, G, Tb, I, 3, 4, 1e-6)
    up = ref.dequant(ref.int_mm(q2, W["up"][0]), s2, W["up"][1], W["up"][2])
    return X1, Tb, I, W, qkv, up


# Rows on both sides of 256-row tile edges, every frame boundary of the
# per-frame modulation (t // 2048), the first and last text rows and the last row.
C5_ROWS = [0, 1, 255, 256, 2047, 2048, 4095, 4096, 6143, 6144, 8191, 8192, 10239, 10240, 12287,
           12288, 12289, 12543, 12544, 12604]


@torch.inference_mode()
def test_c5_ragged_chain_per_frame_rows_match_oracle():
    """T = 12605 (M not a tile multiple), per-frame adaLN rows
    (indices min(t // 2048, 5) for video tokens, 0 for text), out-proj N = 5120
    with the per-token gated-residual epilogue, FFN up N = 20480 + GELU,
    FFN down K = 20480 with the per-token gated residual."""
    g = torch.Generator().manual_seed(20261201 + 4)
    t, x, attn, table, idx, gamma, packed = _c5_inputs(g)
    qkv, x1, x2 = _run_chain(x, attn, table, idx, gamma, packed, "gelu_tanh")
    sel = torch.tensor(C5_ROWS, device="cuda")
    got_qkv, got_x1, got_x2 = (to_np(v.reshape(t, -1).index_select(0, sel)) for v in (qkv, x1, x2))
    X1, Tb, I, W, want_qkv, up = _oracle_front(C5_ROWS, x, attn, table, idx, gamma, packed)
    r = len(C5_ROWS)
    assert np.array_equal(got_qkv, want_qkv), "QKV rows"
    assert np.array_equal(got_x1, X1.reshape(r, D)), "residual after the out-projection"
    q3, s3 = ref.quantize_rows(ref.gelu_tanh(up))
    dn = ref.dequant(ref.int_mm(q3, W["down"][0]), s3, W["down"][1], W["down"][2])
    X2 = ref.gated_residual(X1, dn.reshape(1, r, D), Tb, I, 5).reshape(r, D)
    _assert_rows_close(got_x2, X2, C5_ROWS)


C3_ROWS = [0, 1, 255, 256, 4097, 8191, 8192, 12030, 12287]


@torch.inference_mode()
def test_swiglu_chain_full_size_rows_match_oracle():
    """The reference's own FFN (model/fusion.py:93-97: SwiGLU + INT8 quant, then
    the down projection with the gated residual) at the C3 size: T = 12288,
    D = 5120, up N = 2 * 10240, down K = 10240. SwiGLU's sigmoid uses the
    hardware exp2 / reciprocal, so the block output is compared by tolerance;
    the SwiGLU int8 rows themselves within +-1 LSB."""
    g = torch.Generator().manual_seed(20261201 + 2)
    inner = 10240
    t = 12288
    x = bf16_randn((1, t, D), g, outliers=0.01)
    attn = bf16_randn((1, t, D), g)
    table = (0.1 * torch.randn(1, 6 * D, generator=g)).bfloat16()
    idx = torch.zeros(t, dtype=torch.int64)
    gamma = (1 + 0.05 * torch.randn(D, generator=g)).bfloat16()
    packed = {"to_qkv": _weights(g, 3 * D, D), "to_out": _weights(g, D, D),
              "up": _weights(g, 2 * inner, D), "down": _weights(g, D, inner)}
    qkv, x1, x2 = _run_chain(x, attn, table, idx, gamma, packed, "swiglu")
    sel = torch.tensor(C3_ROWS, device="cuda")
    got_qkv, got_x1, got_x2 = (to_np(v.reshape(t, -1).index_select(0, sel)) for v in (qkv, x1, x2))
    X1, Tb, I, W, want_qkv, up = _oracle_front(C3_ROWS, x, attn, table, idx, gamma, packed)
    r = len(C3_ROWS)
    assert np.array_equal(got_qkv, want_qkv), "QKV rows"
    assert np.array_equal(got_x1, X1.reshape(r, D)), "residual after the out-projection"
    q3, s3 = ref.swiglu_quant(up)
    dn = ref.dequant(ref.int_mm(q3, W["down"][0]), s3, W["down"][1], W["down"][2])
    X2 = ref.gated_residual(X1, dn.reshape(1, r, D), Tb, I, 5).reshape(r, D)
    _assert_rows_close(got_x2, X2, C3_ROWS)
