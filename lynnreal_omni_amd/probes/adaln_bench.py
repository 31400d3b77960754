"""Time the adaLN table kernel against torch's bf16 linear at the C2/C5 shapes.

Usage (on a gfx950 box): python -m lynnreal_omni_amd.probes.adaln_bench
For M time embeddings (1 and 6), K = 5120, N = 6 * 5120: the W8A8 path's
table linear(F.silu(temb).to(bf16)) through lr_adaln_table, and the same
expression in torch (F.silu, then F.linear on hipBLASLt). One JSON line per
M: average time per call (HIP events, current stream) and the algorithmic
HBM rate on the weight, 2 * N * K bytes.
"""
import json

import torch
import torch.nn.functional as F

from lynnreal_omni_amd import kernels


def _time(fn, iters=100):
    for _ in range(5):
        fn()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(iters):
        fn()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) * 1e3 / iters


def main() -> int:
    k, n = 5120, 6 * 5120
    g = torch.Generator(device="cuda").manual_seed(2)
    w = (0.02 * torch.randn(n, k, device="cuda", generator=g)).bfloat16()
    b = (0.1 * torch.randn(n, device="cuda", generator=g)).bfloat16()
    for m in (1, 6):
        temb = torch.randn(m, k, device="cuda", generator=g)
        ours = _time(lambda: kernels.adaln_table(temb, w, b))
        theirs = _time(lambda: F.linear(F.silu(temb).to(torch.bfloat16), w, b))
        gbs = 2 * n * k / (ours * 1e-6) / 1e9
        print(json.dumps({"kernel": "adaln_table", "rows": m, "k": k, "n": n, "us": round(ours, 2),
                          "GB/s": round(gbs, 1), "hbm_frac": round(gbs / 8000, 4),
                          "torch_silu_linear_us": round(theirs, 2)}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
