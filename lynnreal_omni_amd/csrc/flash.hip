// flash.hip - Flash token selection: row gather, residual restore and the
// nearest-anchor search of the selection layout.
//
// Restates model/flash.py:6-33 (spatial_layout: each dropped video row maps to
// its nearest retained row of the same time step) and :71-85 (compress: the
// hidden rows, adaLN indices and rotary rows of the kept tokens are selected
// before the compressed blocks; restore: full + gain * (current - input),
// gathered back through the inverse map, before the first full block).
//
// All three are HBM-bound (the search is a small O(dropped x anchors) pass
// over positions that sit in LDS). Rows are moved as 16-byte chunks by one
// 256-thread block per output row.
#include "lr_device.h"
#include "lr_runtime.h"

namespace lr {
namespace {

constexpr int kThreads = 256;

// -------------------------------------------------------------- gather ----
// dst[o, i, :] = src[o, index[i], :] for rows of `units` 16-byte chunks.
// Indices past the source are clamped (the callers' maps are in range by
// construction; the clamp keeps a bad map inside the buffer).
__global__ __launch_bounds__(kThreads) void gather_rows16(const uint4* __restrict__ src,
                                                          const int64_t* __restrict__ index,
                                                          uint4* __restrict__ dst, int64_t src_rows,
                                                          int64_t dst_rows, int64_t units) {
  const int64_t r = blockIdx.x;  // output row over [outer, dst_rows]
  const int64_t o = r / dst_rows, i = r - o * dst_rows;
  const int64_t s = clamp_index(index[i], src_rows);
  const uint4* from = src + (o * src_rows + s) * units;
  uint4* to = dst + r * units;
  for (int64_t u = threadIdx.x; u < units; u += kThreads) store_nt(to + u, load_nt(from + u));
}

// Any row width: one thread per byte, rows of `width` bytes.
__global__ __launch_bounds__(kThreads) void gather_rows_bytes(const uint8_t* __restrict__ src,
                                                              const int64_t* __restrict__ index,
                                                              uint8_t* __restrict__ dst,
                                                              int64_t src_rows, int64_t dst_rows,
                                                              int64_t width, int64_t total) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= total) return;
  const int64_t r = e / width, c = e - r * width;
  const int64_t o = r / dst_rows, i = r - o * dst_rows;
  const int64_t s = clamp_index(index[i], src_rows);
  dst[e] = src[(o * src_rows + s) * width + c];
}

// ------------------------------------------------------------- restore ----
// out[o, t, c] = bf16(full[o, t, c] + bf16(bf16(cur - inp)[o, inv[t], c] * gain))
// (bf16 tensor ops: each op computes in fp32 and rounds once).
__device__ __forceinline__ float restore1(float full, float cur, float inp, float gain) {
  return full + round_bf(round_bf(cur - inp) * gain);
}

__global__ __launch_bounds__(kThreads) void restore_rows8(const uint4* __restrict__ full,
                                                          const uint4* __restrict__ cur,
                                                          const uint4* __restrict__ inp,
                                                          const int64_t* __restrict__ inverse,
                                                          uint4* __restrict__ out, int64_t out_rows,
                                                          int64_t rows, int64_t compressed,
                                                          int64_t units, float gain) {
  // Consecutive blocks go to different XCDs (round robin over 8). Give each
  // XCD a contiguous range of output rows instead, so that the neighbouring
  // rows that restore from one compressed row share that XCD's L2.
  const int64_t per_xcd = (int64_t)gridDim.x / 8;
  const int64_t r = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (r >= out_rows) return;
  const int64_t o = r / rows, t = r - o * rows;
  const int64_t s = o * compressed + clamp_index(inverse[t], compressed);
  for (int64_t u = threadIdx.x; u < units; u += kThreads) {
    float f[8], c[8], x[8];
    unpack8(load_nt(full + r * units + u), f);
    unpack8(cur[s * units + u], c);
    unpack8(inp[s * units + u], x);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = restore1(f[e], c[e], x[e], gain);
    store_nt(out + r * units + u, pack8(f));
  }
}

__global__ __launch_bounds__(kThreads) void restore_rows_any(const uint16_t* __restrict__ full,
                                                             const uint16_t* __restrict__ cur,
                                                             const uint16_t* __restrict__ inp,
                                                             const int64_t* __restrict__ inverse,
                                                             uint16_t* __restrict__ out,
                                                             int64_t rows, int64_t compressed,
                                                             int64_t width, int64_t total,
                                                             float gain) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= total) return;
  const int64_t r = e / width, c = e - r * width;
  const int64_t o = r / rows, t = r - o * rows;
  const int64_t s = (o * compressed + clamp_index(inverse[t], compressed)) * width + c;
  const float v = restore1(bf_to_f(full[e]), bf_to_f(cur[s]), bf_to_f(inp[s]), gain);
  out[e] = (uint16_t)(pack_bf2(v, 0.0f) & 0xffffu);
}

// ------------------------------------------------------ nearest anchor ----
// For dropped row d, over anchors a in increasing order: skip those whose
// time pos[a, 0] differs from pos[d, 0]; keep the first a with the smallest
// (h_d - h_a)^2 + (w_d - w_a)^2. Coordinates are fp32 (the reference casts
// positions with .float()); the distance is formed in fp64, whose rounding
// lies far below the fp32 spacing of the coordinates, and exact ties (integer
// or dyadic grids) resolve to the first anchor, as torch's argmin does. No
// anchor of the same time leaves a = 0, as argmin over a row of +inf does.
// Then inverse[dropped[d]] = inverse[anchors[a]]. Row numbers past `tokens`
// are clamped, like the gather's indices.
//
// One wave per dropped row: lane l scans anchors l, l + 64, ... of each tile
// of anchor positions staged in LDS for the block's rows, keeping its first
// nearest one, and a wave minimum over (distance, anchor index) then gives
// the first nearest anchor of all.
constexpr int kAnchorTile = 1024;
constexpr int kAnchorRows = kThreads / 64;  // dropped rows per block

__global__ __launch_bounds__(kThreads) void nearest_anchor(const float* __restrict__ pos,
                                                           const int64_t* __restrict__ dropped,
                                                           const int64_t* __restrict__ anchors,
                                                           int64_t* __restrict__ inverse,
                                                           int64_t tokens, int64_t n_dropped,
                                                           int64_t n_anchors) {
  __shared__ float tt[kAnchorTile], th[kAnchorTile], tw[kAnchorTile];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t d = (int64_t)blockIdx.x * kAnchorRows + wave;
  const bool live = d < n_dropped;
  const int64_t row = live ? clamp_index(dropped[d], tokens) : 0;
  const float t0 = live ? pos[3 * row] : 0.0f;
  const double h0 = live ? (double)pos[3 * row + 1] : 0.0;
  const double w0 = live ? (double)pos[3 * row + 2] : 0.0;
  double best = __builtin_inf();
  int64_t best_a = 0;
  for (int64_t base = 0; base < n_anchors; base += kAnchorTile) {
    const int n = (int)min((int64_t)kAnchorTile, n_anchors - base);
    __syncthreads();
    for (int j = threadIdx.x; j < n; j += kThreads) {
      const int64_t a = clamp_index(anchors[base + j], tokens);
      tt[j] = pos[3 * a];
      th[j] = pos[3 * a + 1];
      tw[j] = pos[3 * a + 2];
    }
    __syncthreads();
    for (int j = lane; j < n; j += 64) {
      if (tt[j] != t0) continue;
      const double dh = h0 - (double)th[j], dw = w0 - (double)tw[j];
      const double dist = dh * dh + dw * dw;
      if (dist < best) {
        best = dist;
        best_a = base + j;
      }
    }
  }
  // The first anchor of the smallest distance over the wave; lanes that found
  // none hold (+inf, 0), so a row with no anchor of its time keeps a = 0.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const double od = __shfl_xor(best, off);
    const int64_t oa = __shfl_xor(best_a, off);
    if (od < best || (od == best && oa < best_a)) {
      best = od;
      best_a = oa;
    }
  }
  if (live && lane == 0) inverse[row] = inverse[clamp_index(anchors[best_a], tokens)];
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_gather_rows(const void* src, const int64_t* index, void* dst, int64_t outer,
                              int64_t src_rows, int64_t dst_rows, int64_t row_bytes,
                              void* stream) {
  LR_REQUIRE(outer >= 0 && src_rows >= 0 && dst_rows >= 0 && row_bytes >= 0,
             "gather_rows: negative shape");
  const int64_t rows = outer * dst_rows;
  if (rows == 0 || row_bytes == 0) return LR_OK;
  LR_REQUIRE(src_rows > 0, "gather_rows: index into an empty source");
  LR_REQUIRE(src && index && dst, "gather_rows: null pointer");
  hipStream_t st = as_stream(stream);
  if (row_bytes % 16 == 0 && aligned(src, 16) && aligned(dst, 16)) {
    LR_REQUIRE(rows <= 0x7fffffffLL, "gather_rows: too many rows");
    hipLaunchKernelGGL(gather_rows16, dim3((unsigned)rows), dim3(kThreads), 0, st,
                       (const uint4*)src, index, (uint4*)dst, src_rows, dst_rows, row_bytes / 16);
  } else {
    const int64_t total = rows * row_bytes;
    const int64_t blocks = (total + kThreads - 1) / kThreads;
    LR_REQUIRE(blocks <= 0x7fffffffLL, "gather_rows: too many bytes");
    hipLaunchKernelGGL(gather_rows_bytes, dim3((unsigned)blocks), dim3(kThreads), 0, st,
                       (const uint8_t*)src, index, (uint8_t*)dst, src_rows, dst_rows, row_bytes,
                       total);
  }
  return check_launch("gather_rows");
}

extern "C" int lr_flash_restore(const void* full, const void* current, const void* input,
                                const int64_t* inverse, void* out, int64_t outer, int64_t rows,
                                int64_t compressed_rows, int64_t width, float gain, void* stream) {
  LR_REQUIRE(outer >= 0 && rows >= 0 && compressed_rows >= 0 && width >= 0,
             "flash_restore: negative shape");
  const int64_t out_rows = outer * rows;
  if (out_rows == 0 || width == 0) return LR_OK;
  LR_REQUIRE(compressed_rows > 0, "flash_restore: no compressed rows to restore from");
  LR_REQUIRE(full && current && input && inverse && out, "flash_restore: null pointer");
  hipStream_t st = as_stream(stream);
  if (width % 8 == 0 && aligned(full, 16) && aligned(current, 16) && aligned(input, 16) &&
      aligned(out, 16)) {
    const int64_t blocks = 8 * ((out_rows + 7) / 8);  // a whole number of rows per XCD
    LR_REQUIRE(blocks <= 0x7fffffffLL, "flash_restore: too many rows");
    hipLaunchKernelGGL(restore_rows8, dim3((unsigned)blocks), dim3(kThreads), 0, st,
                       (const uint4*)full, (const uint4*)current, (const uint4*)input, inverse,
                       (uint4*)out, out_rows, rows, compressed_rows, width / 8, gain);
  } else {
    const int64_t total = out_rows * width;
    const int64_t blocks = (total + kThreads - 1) / kThreads;
    LR_REQUIRE(blocks <= 0x7fffffffLL, "flash_restore: too many elements");
    hipLaunchKernelGGL(restore_rows_any, dim3((unsigned)blocks), dim3(kThreads), 0, st,
                       (const uint16_t*)full, (const uint16_t*)current, (const uint16_t*)input,
                       inverse, (uint16_t*)out, rows, compressed_rows, width, total, gain);
  }
  return check_launch("flash_restore");
}

extern "C" int lr_flash_nearest_anchor(const float* positions, int64_t tokens,
                                       const int64_t* dropped, int64_t n_dropped,
                                       const int64_t* anchors, int64_t n_anchors,
                                       int64_t* inverse, void* stream) {
  LR_REQUIRE(tokens >= 0 && n_dropped >= 0 && n_anchors >= 0, "nearest_anchor: negative shape");
  if (n_dropped == 0) return LR_OK;
  LR_REQUIRE(n_anchors > 0 && tokens > 0, "nearest_anchor: dropped rows but no anchors");
  LR_REQUIRE(positions && dropped && anchors && inverse, "nearest_anchor: null pointer");
  const int64_t blocks = (n_dropped + kAnchorRows - 1) / kAnchorRows;
  LR_REQUIRE(blocks <= 0x7fffffffLL, "nearest_anchor: too many rows");
  hipLaunchKernelGGL(nearest_anchor, dim3((unsigned)blocks), dim3(kThreads), 0, as_stream(stream),
                     positions, dropped, anchors, inverse, tokens, n_dropped, n_anchors);
  return check_launch("nearest_anchor");
}
