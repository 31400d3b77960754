"""Time the fused Q/K RMSNorm + RoPE kernel at the C2 shape.

Usage (on a gfx950 box): python -m lynnreal_omni_amd.probes.qk_bench [--tokens T] [--rotary R]
The Q and K inputs are strided views of a fused QKV projection output
[1, T, 3 * heads, head_dim], as model/fusion.py:22-30 produces them. Prints
one JSON line: average launch time (HIP events on the launch stream) and
the algorithmic HBM rate, bytes = 8 * rows * head_dim (Q and K read, Q and K
written, bf16) + 8 * T * rotary_dim (fp32 cos and sin tables).
"""
import argparse
import json

import torch

from lynnreal_omni_amd import kernels


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--tokens", type=int, default=12288)
    p.add_argument("--heads", type=int, default=40)
    p.add_argument("--head-dim", type=int, default=128)
    p.add_argument("--rotary", type=int, default=128)
    p.add_argument("--iters", type=int, default=200)
    a = p.parse_args()
    g = torch.Generator().manual_seed(20261201)
    qkv = torch.randn(1, a.tokens, 3 * a.heads, a.head_dim, generator=g).bfloat16().cuda()
    q, k = qkv[:, :, :a.heads], qkv[:, :, a.heads:2 * a.heads]
    w = (1 + 0.05 * torch.randn(2, a.head_dim, generator=g)).bfloat16().cuda()
    phase = torch.randn(a.tokens, a.rotary, generator=g).cuda()
    rope = (phase.cos(), phase.sin())
    for _ in range(10):
        kernels.qk_norm_rope(q, k, w[0], w[1], rope, 1e-6)
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(a.iters):
        kernels.qk_norm_rope(q, k, w[0], w[1], rope, 1e-6)
    stop.record(stream)
    stop.synchronize()
    us = start.elapsed_time(stop) * 1e3 / a.iters
    rows = a.tokens * a.heads
    nbytes = 8 * rows * a.head_dim + 8 * a.tokens * a.rotary
    gbs = nbytes / (us * 1e-6) / 1e9
    print(json.dumps({"kernel": "qk_norm_rope", "tokens": a.tokens, "heads": a.heads,
                      "head_dim": a.head_dim, "rotary_dim": a.rotary, "us_per_launch": round(us, 2),
                      "algorithmic_bytes": nbytes, "GB/s": round(gbs, 1),
                      "hbm_frac": round(gbs / 8000.0, 4)}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
