"""Time the HBM-bound row kernels of the W8A8 path at the C2/C3 shapes.

Usage (on a gfx950 box):
  python -m lynnreal_omni_amd.probes.row_bench [--tokens T] [--flush]
T = 12288 rows, D = 5120, FFN 20480 (SwiGLU inner 10240). One JSON line per
kernel: time per launch (HIP events on the current stream; back-to-back
launches, or with --flush single launches after a 1 GiB write that evicts
the 256 MB MALL, whose median is reported) and the algorithmic HBM rate
against the 8 TB/s peak, with
bytes counted as the one pass each kernel makes over its rows:
  rms_adaln_quant     3 T D + 4 T      (x in, q out, scales)
  rms_adaln           4 T D            (x in, y out)
  residual_rms_quant  7 T D + 4 T      (x, u in; x' out; q out; scales)
  gated_residual      6 T D            (x, u in; out)
  quantize_rows       3 T K + 4 T
  swiglu_quant        5 T I + 4 T      (P [T, 2I] in; q [T, I] out; scales)
(parameter rows, gamma and table rows, are read once and not counted).
"""
import argparse
import json
import statistics
import types

import torch

from lynnreal_omni_amd import kernels as k


def _time(fn, iters, flush=None):
    """Average us per launch. Without `flush`, back-to-back launches between
    two events. With it (a 1 GiB buffer), the 256 MB MALL is overwritten
    before every launch and each launch is timed on its own: the median of
    those times, with inputs cold in every cache."""
    for _ in range(5):
        fn()
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    if flush is None:
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(iters):
            fn()
        stop.record(stream)
        stop.synchronize()
        return start.elapsed_time(stop) * 1e3 / iters
    times = []
    for _ in range(iters):
        flush.zero_()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        fn()
        stop.record(stream)
        stop.synchronize()
        times.append(start.elapsed_time(stop) * 1e3)
    return statistics.median(times)


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--tokens", type=int, default=12288)
    p.add_argument("--hidden", type=int, default=5120)
    p.add_argument("--ffn", type=int, default=20480)
    p.add_argument("--iters", type=int, default=50)
    p.add_argument("--flush", action="store_true",
                   help="overwrite the MALL before each launch and time launches one by one")
    a = p.parse_args()
    t, d, f = a.tokens, a.hidden, a.ffn
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(1, t, d, device="cuda", generator=g).bfloat16()
    u = torch.randn(1, t, d, device="cuda", generator=g).bfloat16()
    h = torch.randn(t, f, device="cuda", generator=g).bfloat16()
    table = (0.1 * torch.randn(1, 6 * d, device="cuda", generator=g)).bfloat16()
    idx = torch.zeros(t, dtype=torch.int64, device="cuda")
    norm = types.SimpleNamespace(weight=(1 + 0.05 * torch.randn(d, device="cuda", generator=g)).bfloat16(),
                                 eps=1e-6)
    h2 = torch.empty_like(h)
    cases = [
        ("rms_adaln_quant", lambda: k._rms_adaln_quant_int8(x, norm, table, idx, 0, 1), 3 * t * d + 4 * t),
        ("rms_adaln", lambda: k._rms_adaln(x, norm, table, idx, 0, 1), 4 * t * d),
        ("residual_rms_quant", lambda: k.residual_rms_quant(x, u, norm, table, idx), 7 * t * d + 4 * t),
        ("gated_residual", lambda: k._gated_residual(x, u, table, idx, 2), 6 * t * d),
        ("quantize_rows_k%d" % d, lambda: k.quantize_rows(x.view(t, d)), 3 * t * d + 4 * t),
        ("quantize_rows_k%d" % f, lambda: k.quantize_rows(h), 3 * t * f + 4 * t),
        ("swiglu_quant_i%d" % (f // 2), lambda: k._swiglu_quant_int8(h), 5 * t * (f // 2) + 4 * t),
        # the practical streaming ceiling: torch's own device copy of the FFN-wide rows
        ("torch_copy_reference", lambda: h2.copy_(h), 4 * t * f),
    ]
    flush = torch.empty(1 << 30, dtype=torch.uint8, device="cuda") if a.flush else None
    for name, fn, nbytes in cases:
        us = _time(fn, a.iters, flush)
        gbs = nbytes / (us * 1e-6) / 1e9
        print(json.dumps({"kernel": name, "rows": t, "flush": a.flush, "us": round(us, 2), "bytes": nbytes,
                          "GB/s": round(gbs, 1), "hbm_frac": round(gbs / 8000, 4)}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
