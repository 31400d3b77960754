"""Write the golden fixtures of the W8A8 path into tests/golden/.

The reference commits no golden vectors for this path, so the expected
outputs here come from oracle/torch_path.py: the reference's torch path
(model/int8.py:60-68, model/int8_gemm.py:84-92) and the Triton kernels'
arithmetic (model/kernels.py) written with torch's own CPU operators. They
are independent of the C oracle, which the CPU tests check against them.

Run from the repo root:  python tests/golden/make_golden.py
Inputs are drawn from torch.Generator().manual_seed(...) on the CPU, so the
file contents are reproducible.

golden_small.npz  full inputs and outputs of small cases (bf16 as uint16)
golden_kat.json   sha256 of the bf16 outputs of the reference's install-time
                  GEMM check shapes (script/precompile.py:50): inputs are
                  regenerated from the seed, outputs compared by digest
"""
from __future__ import annotations

import hashlib
import json
import pathlib
import sys

import numpy as np
import torch

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from helpers import bf16_randn, to_np  # noqa: E402
from oracle import torch_path as tp  # noqa: E402

HERE = pathlib.Path(__file__).resolve().parent

# (M, N, K) of script/precompile.py:50.
KAT_SHAPES = [(32, 21504, 5376), (32, 5376, 7168), (32, 28672, 5376), (32, 5376, 14336)]


def kat_inputs(m, n, k, seed=219):
    """Random int8 A [M,K], W [N,K] and rand/127 scales, as the reference's
    check draws them (script/precompile.py:55-59), from a CPU generator."""
    g = torch.Generator().manual_seed(seed + m + n + k)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
    rs = torch.rand(m, 1, generator=g) / 127
    cs = torch.rand(1, n, generator=g) / 127
    return a, w, rs, cs


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(to_np(t).tobytes()).hexdigest()


def small_cases() -> dict[str, np.ndarray]:
    g = torch.Generator().manual_seed(20261201)
    out: dict[str, np.ndarray] = {}
    # quantizer: 1% outlier channels x20, a zero row, a ragged width
    x = bf16_randn((8, 5120), g, outliers=0.01)
    x[3] = 0
    q, s = tp.quantize(x)
    out.update(quant_x=to_np(x), quant_q=q.numpy(), quant_s=s.reshape(-1).numpy())
    x = bf16_randn((5, 317), g)
    q, s = tp.quantize(x)
    out.update(quant317_x=to_np(x), quant317_q=q.numpy(), quant317_s=s.reshape(-1).numpy())
    # W8A8 linear with bias: M not a tile multiple
    a = bf16_randn((45, 256), g, outliers=0.01)
    w = torch.randint(-127, 128, (96, 256), dtype=torch.int8, generator=g)
    ws = torch.rand(96, generator=g) * 4e-3 + 1e-3
    bias = (torch.randn(96, generator=g) * 0.02).bfloat16()
    qa, sa = tp.quantize(a)
    acc = tp.int_mm(qa, w)
    y = tp.epilogue(acc, sa, ws, bias)
    out.update(lin_x=to_np(a), lin_w=w.numpy(), lin_ws=ws.numpy(), lin_bias=to_np(bias),
               lin_q=qa.numpy(), lin_s=sa.reshape(-1).numpy(), lin_acc=acc.numpy(), lin_y=to_np(y))
    # fused norm / modulate with a per-token table (R = 3), gated residuals
    hidden = 512
    x = bf16_randn((2, 12, hidden), g, outliers=0.01)
    u = bf16_randn((2, 12, hidden), g)
    wn = (1 + 0.05 * torch.randn(hidden, generator=g)).bfloat16()
    table = bf16_randn((3, 6 * hidden), g, scale=0.1)
    idx = torch.tensor([0, 0, 1, 1, 2, 2, 0, 1, 2, 2, 1, 0])
    y01 = tp.rms_adaln(x, wn, table, idx, 0, 1, 1e-6)
    r2 = tp.gated_residual(x, u, table, idx, 2)
    y34 = tp.rms_adaln(r2, wn, table, idx, 3, 4, 1e-6)
    q34, s34 = tp.quantize(y34.reshape(-1, hidden))
    r5 = tp.gated_residual(x, u, table, idx, 5)
    out.update(norm_x=to_np(x), norm_u=to_np(u), norm_w=to_np(wn), norm_table=to_np(table),
               norm_idx=idx.numpy(), norm_y01=to_np(y01), norm_r2=to_np(r2), norm_y34=to_np(y34),
               norm_q34=q34.numpy(), norm_s34=s34.reshape(-1).numpy(), norm_r5=to_np(r5))
    # activations
    p = bf16_randn((6, 2 * 160), g, scale=2.0)
    out.update(swiglu_p=to_np(p), swiglu_y=to_np(tp.swiglu(p)))
    v = torch.linspace(-8, 8, 4096).bfloat16()
    out.update(gelu_x=to_np(v), gelu_y=to_np(tp.gelu_tanh(v)))
    return out


def kat_digests() -> dict:
    result = {}
    for m, n, k in KAT_SHAPES:
        a, w, rs, cs = kat_inputs(m, n, k)
        acc = tp.int_mm(a, w)
        y = tp.epilogue(acc, rs, cs)
        result[f"{m}x{n}x{k}"] = {"acc_sha256": hashlib.sha256(acc.numpy().tobytes()).hexdigest(),
                                  "y_sha256": digest(y)}
    return result


def main():
    np.savez_compressed(HERE / "golden_small.npz", **small_cases())
    (HERE / "golden_kat.json").write_text(json.dumps(kat_digests(), indent=1) + "\n")
    print("wrote", HERE / "golden_small.npz", HERE / "golden_kat.json")


if __name__ == "__main__":
    main()
