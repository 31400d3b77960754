"""Time the Flash token-selection kernels on a C5-like layout.

Usage (on a gfx950 box): python -m lynnreal_omni_amd.probes.flash_bench [--frames F]
Layout: `--text` text rows, then `--frames` frames of a `--height` x `--width`
video grid, hidden width D. Prints one JSON line: average launch time (HIP
events on the launch stream) of
  layout   flash.spatial_layout (torch bookkeeping + nearest-anchor kernel)
  gather   hidden rows of the kept tokens, bytes 2 * 2 * kept * D
  restore  full + gain * (current - input)[inverse], bytes
           2 * T * D (full) + 2 * 2 * kept * D (current, input) + 2 * T * D (out)
with the algorithmic HBM rate of the last two.
"""
import argparse
import json

import torch

from lynnreal_omni_amd import flash


def _time(fn, iters):
    for _ in range(3):
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
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--frames", type=int, default=6)
    p.add_argument("--height", type=int, default=32)
    p.add_argument("--width", type=int, default=64)
    p.add_argument("--text", type=int, default=317)
    p.add_argument("--hidden", type=int, default=5120)
    p.add_argument("--iters", type=int, default=50)
    a = p.parse_args()
    t_h = torch.arange(a.frames, dtype=torch.float64).repeat_interleave(a.height * a.width)
    hh = torch.arange(a.height, dtype=torch.float64).repeat_interleave(a.width).repeat(a.frames)
    ww = torch.arange(a.width, dtype=torch.float64).repeat(a.frames * a.height)
    video = torch.stack([t_h, hh, ww], 1)
    text = torch.stack([torch.arange(a.text, dtype=torch.float64), torch.zeros(a.text),
                        torch.zeros(a.text)], 1)
    pos = torch.cat([text, video]).cuda()
    tags = torch.cat([torch.ones(a.text, dtype=torch.long),
                      torch.zeros(video.shape[0], dtype=torch.long)]).cuda()
    tokens = pos.shape[0]
    keep, inverse = flash.spatial_layout(pos, tags)
    kept = keep.numel()
    g = torch.Generator(device="cuda").manual_seed(1)
    full = torch.randn(1, tokens, a.hidden, device="cuda", generator=g).bfloat16()
    cur = torch.randn(1, kept, a.hidden, device="cuda", generator=g).bfloat16()
    inp = torch.randn(1, kept, a.hidden, device="cuda", generator=g).bfloat16()
    layout_us = _time(lambda: flash.spatial_layout(pos, tags), max(5, a.iters // 10))
    gather_us = _time(lambda: flash.gather_rows(full, keep, 1), a.iters)
    restore_us = _time(lambda: flash.restore(full, cur, inp, inverse, 1.0), a.iters)
    gather_bytes = 4 * kept * a.hidden
    restore_bytes = 4 * tokens * a.hidden + 4 * kept * a.hidden
    print(json.dumps({
        "tokens": tokens, "kept": kept, "hidden": a.hidden,
        "layout_us": round(layout_us, 1),
        "gather_us": round(gather_us, 2), "gather_GBs": round(gather_bytes / gather_us / 1e3, 1),
        "restore_us": round(restore_us, 2), "restore_GBs": round(restore_bytes / restore_us / 1e3, 1),
    }), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
