// norm.hip - fused RMSNorm + adaLN modulate (+ gated residual) (+ INT8 quant).
//
// Restates model/kernels.py:48-128 (_rms_adaln_kernel and
// _rms_adaln_quant_int8_kernel, incl. its WITH_RESIDUAL branch :101-105).
//
// Main kernel: one wave per row (token), four rows per 256-thread block, no
// block barriers. Lane l holds 16-byte chunks l, l+64, ... of the row in
// registers from the first read to the last write, so HBM sees each byte once:
//   rms_adaln            2 B in + 2 B out per element
//   rms_adaln_quant      2 B in + 1 B out per element (+4 B/row)
//   residual_rms_quant   4 B in + 3 B out per element (+4 B/row)
// gamma and the table rows are shared by all rows and come from L2. The
// arithmetic is VALU-bound at these byte counts, so bf16 roundings are done
// two elements per v_cvt_pk_bf16_f32.
//
// The sum of squares uses one fixed order (8-element chunks, chunk j into
// slot j % 256, slots combined by a pairwise tree; see lynnreal_amd.h), so a
// CPU restatement reproduces it bit for bit. In the wave kernel lane l owns
// slots l, l+64, l+128, l+192 (chunk l + 64m goes to slot l + 64(m % 4)); the
// tree's two top levels are then lane-local and the rest is the butterfly.
// The reference's Triton kernel sums in its own tree order with an
// approximate rsqrt; against it the bf16 outputs agree to a bf16 ulp.
//
// Rows wider than the wave kernel holds (hidden > 8192) or unaligned rows use
// a one-row-per-block kernel with the same arithmetic.
#include "lr_device.h"
#include "lr_runtime.h"

namespace lr {
namespace {

constexpr int kThreads = 256;

struct NormArgs {
  const uint16_t* x;
  const uint16_t* u;
  const uint16_t* w;
  const uint16_t* table;
  const int64_t* indices;
  uint16_t* out;
  uint16_t* resid_out;
  int8_t* q;
  float* scales;
  int64_t sequence, hidden, table_rows, table_width;
  int shift_slot, scale_slot, gate_slot;
  float eps;
};

// Loads chunk c (elements 8c .. 8c+7) of a bf16 row of length n; elements at
// or past n read as zero.
template <bool VEC>
__device__ __forceinline__ void load8(const uint16_t* row, int64_t c, int64_t n, float f[8]) {
  if (VEC) {
    unpack8(*reinterpret_cast<const uint4*>(row + 8 * c), f);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t i = 8 * c + e;
      f[e] = i < n ? bf_to_f(row[i]) : 0.0f;
    }
  }
}

template <bool VEC>
__device__ __forceinline__ void store8(uint16_t* row, int64_t c, int64_t n, const float f[8]) {
  if (VEC) {
    *reinterpret_cast<uint4*>(row + 8 * c) = pack8(f);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t i = 8 * c + e;
      if (i < n) row[i] = (uint16_t)(pack_bf2(f[e], 0.0f) & 0xffffu);
    }
  }
}

template <bool VEC>
__device__ __forceinline__ void store8_i8(int8_t* row, int64_t c, int64_t n, const float f[8],
                                          float s, float inv) {
  if (VEC) {
    *reinterpret_cast<uint2*>(row + 8 * c) = quant8(f, s, inv);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t i = 8 * c + e;
      if (i < n) row[i] = (int8_t)quant_one(f[e], s, inv);
    }
  }
}

template <int CPT, bool VEC, bool RESID, bool QUANT>
__global__ __launch_bounds__(kThreads) void rms_adaln_kernel(NormArgs p) {
  __shared__ float red[kThreads];
  const int64_t row = blockIdx.x;
  const int64_t H = p.hidden;
  const int64_t chunks = (H + 7) / 8;
  const int64_t tr = clamp_index(p.indices[row % p.sequence], p.table_rows);
  const uint16_t* trow = p.table + tr * p.table_width;
  const uint16_t* xrow = p.x + row * H;

  float v[CPT][8];
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + i * kThreads;
    if (c < chunks) {
      load8<VEC>(xrow, c, H, v[i]);
      if (RESID) {
        // x' = bf16(x + bf16(gate * u)), gate = table slot 2 (kernels.py:101-105)
        float uu[8], gg[8];
        load8<VEC>(p.u + row * H, c, H, uu);
        load8<VEC>(trow + 2 * H, c, H, gg);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = round_bf(v[i][e] + round_bf(gg[e] * uu[e]));
        store8<VEC>(p.resid_out + row * H, c, H, v[i]);
      }
      // A bf16 square is exact in fp32, so fma(x, x, s) is s + x*x rounded once.
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(v[i][e], v[i][e], acc);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
    }
  }
  const float ss = block256_tree_sum(acc, red);
  float ms = ss / (float)H;
  ms = ms + p.eps;
  const float rr = 1.0f / __builtin_sqrtf(ms);

  const uint16_t* shift = trow + (int64_t)p.shift_slot * H;
  const uint16_t* scale = trow + (int64_t)p.scale_slot * H;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + i * kThreads;
    if (c < chunks) {
      float w8[8], sc8[8], sh8[8];
      load8<VEC>(p.w, c, H, w8);
      load8<VEC>(scale, c, H, sc8);
      load8<VEC>(shift, c, H, sh8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float n = round_bf((v[i][e] * rr) * w8[e]);
        const float m = round_bf(n * round_bf(1.0f + sc8[e]));
        const float y = round_bf(m + sh8[e]);
        v[i][e] = y;
        amax = fmaxf(amax, __builtin_fabsf(y));
      }
      if (!QUANT) store8<VEC>(p.out + row * H, c, H, v[i]);
    }
  }
  if (QUANT) {
    __syncthreads();  // every thread is done reading `red` from the sum
    amax = block256_max(amax, red);
    const float s = quant_scale(amax);
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int64_t c = threadIdx.x + i * kThreads;
      if (c < chunks) store8_i8<VEC>(p.q + row * H, c, H, v[i], s, inv);
    }
    if (threadIdx.x == 0) p.scales[row] = s;
  }
}

// ------------------------------------------------ streaming kernel ----
// A persistent grid (as many blocks as are resident) in which block
// b owns rows [b * per_block, (b + 1) * per_block). At block start, gamma and
// the modulation rows of the slice's first token are expanded into LDS as
// fp32: gamma, bf16(1 + scale), shift and (residual) gate. Wave w of W then
// streams rows start + w, start + w + W, ... and reads the parameters from
// LDS (their waits, lgkmcnt, do not wait for row loads in flight). A slice
// that spans two runs of equal table rows (a frame boundary of per-frame
// modulation) processes the first run, restages the second run's row and
// processes the rest; a slice with more runs reads its parameters from
// global memory. Slices are ceil(rows / resident blocks) rows, so every CU
// gets the same share whatever the frame length.
// Waves per block: 16 (four per SIMD, one row per wave at a time) for rows up
// to 5120 wide without a residual, else 8 (two rows per wave, the next one's
// loads in flight). The LDS block is per block, so more waves per block share it.
template <int CPL, bool RESID>
constexpr int stream_waves() { return (RESID || CPL > 10) ? 8 : 16; }

// Rows up to 5120 wide without a residual: one row in registers per wave and
// four waves per SIMD (108 VGPRs) hide the loads better than two rows per
// wave at three waves per SIMD (measured 2% faster on the C2 shape).
template <int CPL, bool RESID>
constexpr bool single_buffer() { return !RESID && CPL <= 10; }

// LDS: parameter array a (0 gamma, 1 bf16(1 + scale), 2 shift, 3 gate),
// chunk c, half h (elements 8c + 4h .. 8c + 4h + 3) at float4 (2a + h) * cap + c,
// so that the 64 lanes of a wave read 64 consecutive float4s.
template <int CPL, bool RESID>
struct RowRegs {
  uint4 x[CPL];
  uint4 u[RESID ? CPL : 1];
};

// live = false loads zeros through a zero-size descriptor without touching
// memory. Callers issue the next row's loads unconditionally this way: a load
// under a branch makes the compiler wait for every outstanding load where
// the paths join (vmcnt(0)), which would wait for the prefetched row too.
template <int CPL, bool RESID>
__device__ __forceinline__ void load_row(const NormArgs& p, int64_t row, RowRegs<CPL, RESID>& r,
                                         bool live = true) {
  const int lane = threadIdx.x & 63;
  const int64_t base = (live ? row : 0) * p.hidden;
  const int64_t bytes = live ? 2 * p.hidden : 0;
  const auto xr = row_rsrc(p.x + base, bytes);
#pragma unroll
  for (int m = 0; m < CPL; ++m) r.x[m] = buf_load16(xr, 16u * lane, 1024u * m);
  if (RESID) {
    const auto ur = row_rsrc(p.u + base, bytes);
#pragma unroll
    for (int m = 0; m < CPL; ++m) r.u[m] = buf_load16(ur, 16u * lane, 1024u * m);
  }
}

// The 8 fp32 parameters of array a for chunk c, from LDS or from the table
// row `trow` in global memory. Past the row end gamma, shift and gate read as
// 0 and bf16(1 + scale) as 1, which keeps those lanes' outputs at zero.
template <bool FROM_LDS>
__device__ __forceinline__ void params8(const NormArgs& p, const uint16_t* trow,
                                        const float4* lds, int cap, int a, int c, float f[8]) {
  if (FROM_LDS) {
    const float4 lo = lds[(2 * a) * cap + c], hi = lds[(2 * a + 1) * cap + c];
    f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
    f[4] = hi.x; f[5] = hi.y; f[6] = hi.z; f[7] = hi.w;
  } else {
    const uint16_t* src = a == 0 ? p.w
                        : trow + (int64_t)(a == 1 ? p.scale_slot : (a == 2 ? p.shift_slot : 2)) *
                                     p.hidden;
    unpack8(buf_load16_reused(row_rsrc(src, 2 * p.hidden), 16u * (c & 63), 16u * (c & ~63)), f);
    if (a == 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = round_bf(1.0f + f[e]);
    }
  }
}

// Lanes past the row end hold zeros throughout (x and u read as zero, and
// the parameters keep them there), so they add nothing to the sums and maxima,
// and their stores fall outside the row's buffer range.
template <int CPL, bool RESID, bool QUANT, bool FROM_LDS>
__device__ __forceinline__ void norm_row(const NormArgs& p, int64_t row, const uint16_t* trow,
                                         const float4* lds, RowRegs<CPL, RESID>& r) {
  constexpr int cap = 64 * CPL;
  const int lane = threadIdx.x & 63;
  const int64_t H = p.hidden;
  if (RESID) {
    // x' = bf16(x + bf16(gate * u)), gate = table slot 2 (kernels.py:101-105)
    const auto orow = row_rsrc(p.resid_out + row * H, 2 * H);
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int c = lane + 64 * m;
      float g[8], xf[8], uf[8];
      params8<FROM_LDS>(p, trow, lds, cap, 3, c, g);
      unpack8(r.x[m], xf);
      unpack8(r.u[m], uf);
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[e] = xf[e] + round_bf(g[e] * uf[e]);
      r.x[m] = pack8(xf);
      buf_store16(orow, 16u * lane, 1024u * m, r.x[m]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Lane l's slots l + 64k accumulate chunks m = k, k+4, k+8, ... in order.
  // A bf16 square is exact in fp32, so fma(x, x, s) is s + x*x rounded once.
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    float f[8];
    unpack8(r.x[m], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m & 3] = __builtin_fmaf(f[e], f[e], acc[m & 3]);
  }
  const float ss = wave_tree_sum((acc[0] + acc[2]) + (acc[1] + acc[3]));
  float ms = ss / (float)H;
  ms = ms + p.eps;
  const float rr = 1.0f / __builtin_sqrtf(ms);
  // Keep the row packed across the reduction: unpacking it again below costs
  // one instruction per element, holding it unpacked doubles the registers.
#pragma unroll
  for (int m = 0; m < CPL; ++m) opaque(r.x[m]);

  // Chunk by chunk, with chunk m + 1's parameters read while chunk m computes;
  // the scheduling barriers keep the compiler from hoisting every chunk's reads
  // (which would need 24 registers per chunk).
  const auto orow = row_rsrc(p.out + row * H, 2 * H);
  float amax = 0.0f;
  float nw[8], nmod[8], nsh[8];
  params8<FROM_LDS>(p, trow, lds, cap, 0, lane, nw);
  params8<FROM_LDS>(p, trow, lds, cap, 1, lane, nmod);
  params8<FROM_LDS>(p, trow, lds, cap, 2, lane, nsh);
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    const int c = lane + 64 * m;
    float w[8], mod[8], sh[8], xf[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = nw[e], mod[e] = nmod[e], sh[e] = nsh[e];
    if (m + 1 < CPL) {
      params8<FROM_LDS>(p, trow, lds, cap, 0, c + 64, nw);
      params8<FROM_LDS>(p, trow, lds, cap, 1, c + 64, nmod);
      params8<FROM_LDS>(p, trow, lds, cap, 2, c + 64, nsh);
    }
    unpack8(r.x[m], xf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float n = round_bf((xf[e] * rr) * w[e]);
      const float t = round_bf(n * mod[e]);
      xf[e] = t + sh[e];
      // bf16 rounding is monotonic and odd, so max |bf16(y)| = bf16(max |y|).
      amax = fmaxf(amax, __builtin_fabsf(xf[e]));
    }
    r.x[m] = pack8(xf);
    if (!QUANT) buf_store16(orow, 16u * lane, 1024u * m, r.x[m]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (QUANT) {
#pragma unroll
    for (int m = 0; m < CPL; ++m) opaque(r.x[m]);  // as above, for y
    const float s = quant_scale(wave_max(round_bf(amax)));
    const float inv = 1.0f / s;
    const auto qrow = row_rsrc(p.q + row * H, H);
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      buf_store8(qrow, 8u * lane, 512u * m, quant8_bf(r.x[m], s, inv));
      __builtin_amdgcn_sched_barrier(0);
    }
    if (lane == 0) p.scales[row] = s;
  }
}

// One row of the single-buffer path (no residual, parameters in LDS), with
// the row unpacked once into fp32 registers and normalized in place: the
// sum of squares, the normalization and the quantizer read the same floats,
// which saves two unpacks and a pack per element over norm_row (15.5 instead
// of 17.4 VALU instructions per element for the quantizing 5120-wide row,
// 118-122 VGPRs, still four waves per SIMD; 39 -> 37.7 us at 12288 rows).
// The scheduling barriers keep each chunk's parameter reads next to its
// arithmetic (hoisting them all would spill).
template <int CPL, bool QUANT>
__device__ __forceinline__ void norm_row_f32(const NormArgs& p, int64_t row, const float4* lds,
                                             RowRegs<CPL, false>& r) {
  constexpr int cap = 64 * CPL;
  const int lane = threadIdx.x & 63;
  const int64_t H = p.hidden;
  float f[CPL][8];
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    unpack8(r.x[m], f[m]);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m & 3] = __builtin_fmaf(f[m][e], f[m][e], acc[m & 3]);
    __builtin_amdgcn_sched_barrier(0);
  }
  const float ss = wave_tree_sum((acc[0] + acc[2]) + (acc[1] + acc[3]));
  float ms = ss / (float)H;
  ms = ms + p.eps;
  const float rr = 1.0f / __builtin_sqrtf(ms);
  float amax = 0.0f;
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    const int c = lane + 64 * m;
    float w[8], mod[8], sh[8];
    params8<true>(p, nullptr, lds, cap, 0, c, w);
    params8<true>(p, nullptr, lds, cap, 1, c, mod);
    params8<true>(p, nullptr, lds, cap, 2, c, sh);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float n = round_bf((f[m][e] * rr) * w[e]);
      const float t = round_bf(n * mod[e]);
      f[m][e] = round_bf(t + sh[e]);
      amax = fmaxf(amax, __builtin_fabsf(f[m][e]));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (QUANT) {
    const float rmax = wave_max(amax);
    const float s = quant_scale(rmax);
    const float inv = 1.0f / s;
    const auto qrow = row_rsrc(p.q + row * H, H);
    // Rows below 2^80 (all real activations) take the three-operation quotient.
    if (__builtin_amdgcn_readfirstlane(rmax < 0x1p80f ? 1 : 0)) {
      const float lo = quant_lo(s, inv);
#pragma unroll
      for (int m = 0; m < CPL; ++m) {
        buf_store8(qrow, 8u * lane, 512u * m, quant8_split(f[m], inv, lo));
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int m = 0; m < CPL; ++m) {
        buf_store8(qrow, 8u * lane, 512u * m, quant8(f[m], s, inv));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (lane == 0) p.scales[row] = s;
  } else {
    const auto orow = row_rsrc(p.out + row * H, 2 * H);
#pragma unroll
    for (int m = 0; m < CPL; ++m) buf_store16(orow, 16u * lane, 1024u * m, pack8(f[m]));
  }
}

// Expands the parameters of table row tr into LDS (every thread of the block
// takes part).
template <int CPL, bool RESID, int THREADS>
__device__ __forceinline__ void stage_params(const NormArgs& p, float4* lds, int64_t tr) {
  constexpr int cap = 64 * CPL;
  const uint16_t* trow = p.table + tr * p.table_width;
  for (int c = threadIdx.x; c < cap; c += THREADS) {
    const int na = RESID ? 4 : 3;
    for (int a = 0; a < na; ++a) {
      float f[8];
      params8<false>(p, trow, nullptr, cap, a, c, f);
      lds[(2 * a) * cap + c] = make_float4(f[0], f[1], f[2], f[3]);
      lds[(2 * a + 1) * cap + c] = make_float4(f[4], f[5], f[6], f[7]);
    }
  }
}

// Rows [lo, hi) of the block's slice with the parameters staged in LDS; wave
// w takes rows lo + w, lo + w + WAVES, ...
template <int CPL, bool RESID, bool QUANT, int WAVES>
__device__ __forceinline__ void run_rows(const NormArgs& p, const float4* lds, int64_t lo,
                                         int64_t hi, int wave) {
  int64_t row = lo + wave;
  if constexpr (single_buffer<CPL, RESID>()) {
    RowRegs<CPL, RESID> r1;
    for (; row < hi; row += WAVES) {
      load_row(p, row, r1);
      norm_row_f32<CPL, QUANT>(p, row, lds, r1);
    }
  } else {
    RowRegs<CPL, RESID> ra, rb;
    if (row >= hi) return;
    load_row(p, row, ra);
    while (true) {
      const int64_t next = row + WAVES;
      load_row(p, next, rb, next < hi);  // zeros past the range, no memory access
      norm_row<CPL, RESID, QUANT, true>(p, row, nullptr, lds, ra);
      row = next;
      if (row >= hi) break;
      const int64_t after = row + WAVES;
      load_row(p, after, ra, after < hi);
      norm_row<CPL, RESID, QUANT, true>(p, row, nullptr, lds, rb);
      row = after;
      if (row >= hi) break;
    }
  }
}

template <int CPL, bool RESID, bool QUANT>
__global__ __launch_bounds__((64 * stream_waves<CPL, RESID>())) void rms_adaln_stream(
    NormArgs p, int64_t rows, int64_t per_block) {
  constexpr int kStreamWaves = stream_waves<CPL, RESID>();
  constexpr int kStreamThreads = 64 * kStreamWaves;
  constexpr int cap = 64 * CPL;
  __shared__ float4 lds[(RESID ? 8 : 6) * cap];
  __shared__ int first_other;
  const int64_t start = (int64_t)blockIdx.x * per_block;
  const int64_t end = start + per_block < rows ? start + per_block : rows;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t tr_first = clamp_index(p.indices[start % p.sequence], p.table_rows);
  stage_params<CPL, RESID, kStreamThreads>(p, lds, tr_first);
  if (p.table_rows == 1) {
    // One table row: every row of the slice uses the staged parameters.
    __syncthreads();
    run_rows<CPL, RESID, QUANT, kStreamWaves>(p, lds, start, end, wave);
    return;
  }
  // The slice is one run of equal table rows, two runs (a frame boundary of
  // per-frame modulation), or mixed. split = the first row of the second run.
  if (threadIdx.x == 0) first_other = (int)(end - start);
  __syncthreads();
  for (int64_t r = start + threadIdx.x; r < end; r += kStreamThreads) {
    if (clamp_index(p.indices[r % p.sequence], p.table_rows) != tr_first) {
      atomicMin(&first_other, (int)(r - start));
      break;
    }
  }
  __syncthreads();
  const int64_t split = start + __builtin_amdgcn_readfirstlane(first_other);
  if (split == end) {
    run_rows<CPL, RESID, QUANT, kStreamWaves>(p, lds, start, end, wave);
    return;
  }
  const int64_t tr_second = clamp_index(p.indices[split % p.sequence], p.table_rows);
  int second_run = 1;
  for (int64_t r = split + threadIdx.x; r < end; r += kStreamThreads)
    second_run &= clamp_index(p.indices[r % p.sequence], p.table_rows) == tr_second;
  if (__syncthreads_and(second_run)) {
    run_rows<CPL, RESID, QUANT, kStreamWaves>(p, lds, start, split, wave);
    __syncthreads();  // every wave is done with the first run's parameters
    stage_params<CPL, RESID, kStreamThreads>(p, lds, tr_second);
    __syncthreads();
    run_rows<CPL, RESID, QUANT, kStreamWaves>(p, lds, split, end, wave);
    return;
  }
  // Mixed table rows: parameters from global memory, one row at a time.
  RowRegs<CPL, RESID> rg;
  for (int64_t row = start + wave; row < end; row += kStreamWaves) {
    load_row(p, row, rg);
    const int64_t tr = clamp_index(p.indices[row % p.sequence], p.table_rows);
    norm_row<CPL, RESID, QUANT, false>(p, row, p.table + tr * p.table_width, nullptr, rg);
  }
}

template <int CPL, bool RESID, bool QUANT>
void launch_stream(const NormArgs& p, int64_t rows, hipStream_t st) {
  constexpr int kStreamWaves = stream_waves<CPL, RESID>();
  constexpr int kStreamThreads = 64 * kStreamWaves;
  const auto kernel = rms_adaln_stream<CPL, RESID, QUANT>;
  static int resident = 0;  // blocks per CU; the same for every gfx950 device
  if (resident == 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kernel),
                                                     kStreamThreads, 0) != hipSuccess || nb < 1) {
      (void)hipGetLastError();
      nb = 1;
    }
    resident = nb;
  }
  const int64_t slots = (int64_t)compute_units() * resident;
  const int64_t per_block = (rows + slots - 1) / slots;
  const int64_t grid = (rows + per_block - 1) / per_block;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kStreamThreads), 0, st, p, rows,
                     per_block);
}

// Rows up to 5120 wide (8192 without quantization) stay in registers without
// spilling; wider rows take the one-row-per-block kernel.
template <bool RESID, bool QUANT>
bool launch_norm_stream(const NormArgs& p, int64_t rows, hipStream_t st) {
  const int64_t need = (p.hidden / 8 + 63) / 64;
  if (need <= 1) launch_stream<1, RESID, QUANT>(p, rows, st);
  else if (need <= 2) launch_stream<2, RESID, QUANT>(p, rows, st);
  else if (need <= 4) launch_stream<4, RESID, QUANT>(p, rows, st);
  else if (need <= 6) launch_stream<6, RESID, QUANT>(p, rows, st);
  else if (need <= 8) launch_stream<8, RESID, QUANT>(p, rows, st);
  else if (need <= 10) launch_stream<10, RESID, QUANT>(p, rows, st);
  else if (QUANT) return false;
  else if (need <= 12) launch_stream<12, false, false>(p, rows, st);
  else if (need <= 16) launch_stream<16, false, false>(p, rows, st);
  else return false;
  return true;
}

template <bool RESID, bool QUANT>
int launch_norm(const NormArgs& p, int64_t rows, bool vec, hipStream_t st) {
  if (vec && launch_norm_stream<RESID, QUANT>(p, rows, st)) return check_launch("rms_adaln");
  const int64_t chunks = (p.hidden + 7) / 8;
  const int64_t need = (chunks + kThreads - 1) / kThreads;
  if (need > 16)
    return fail(LR_EUNSUPPORTED, "rms_adaln: hidden=%lld not supported (max %d)",
                (long long)p.hidden, 16 * 8 * kThreads);
#define LR_NORM_LAUNCH(C)                                                                   \
  do {                                                                                      \
    if (vec)                                                                                \
      hipLaunchKernelGGL((rms_adaln_kernel<C, true, RESID, QUANT>), dim3((unsigned)rows),   \
                         dim3(kThreads), 0, st, p);                                         \
    else                                                                                    \
      hipLaunchKernelGGL((rms_adaln_kernel<C, false, RESID, QUANT>), dim3((unsigned)rows),  \
                         dim3(kThreads), 0, st, p);                                         \
  } while (0)
  if (need <= 1) LR_NORM_LAUNCH(1);
  else if (need <= 2) LR_NORM_LAUNCH(2);
  else if (need <= 3) LR_NORM_LAUNCH(3);
  else if (need <= 4) LR_NORM_LAUNCH(4);
  else if (need <= 8) LR_NORM_LAUNCH(8);
  else LR_NORM_LAUNCH(16);
#undef LR_NORM_LAUNCH
  return check_launch("rms_adaln");
}

int check_common(const NormArgs& p, int64_t rows, int slots_needed) {
  LR_REQUIRE(rows >= 0 && p.hidden > 0 && p.sequence > 0, "rms_adaln: bad shape");
  LR_REQUIRE(rows <= 0x7fffffffLL, "rms_adaln: too many rows");
  LR_REQUIRE(p.x && p.w && p.table && p.indices, "rms_adaln: null pointer");
  LR_REQUIRE(p.table_rows > 0, "rms_adaln: empty table");
  LR_REQUIRE(p.shift_slot >= 0 && p.scale_slot >= 0 && p.gate_slot >= 0,
             "rms_adaln: negative slot");
  const int64_t top = (int64_t)(slots_needed) * p.hidden;
  LR_REQUIRE(top <= p.table_width,
             "rms_adaln: table width %lld too small for slot %d of hidden %lld",
             (long long)p.table_width, slots_needed - 1, (long long)p.hidden);
  return LR_OK;
}

bool vec_ok(const NormArgs& p) {
  bool ok = p.hidden % 8 == 0 && p.table_width % 8 == 0 && aligned(p.x, 16) &&
            aligned(p.w, 16) && aligned(p.table, 16);
  if (p.u) ok = ok && aligned(p.u, 16);
  if (p.out) ok = ok && aligned(p.out, 16);
  if (p.resid_out) ok = ok && aligned(p.resid_out, 16);
  if (p.q) ok = ok && aligned(p.q, 8);
  return ok;
}

int max_slot(int a, int b) { return (a > b ? a : b) + 1; }

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_rms_adaln(const void* x, const void* weight, const void* table,
                            const int64_t* indices, void* out, int64_t rows, int64_t sequence,
                            int64_t hidden, int64_t table_rows, int64_t table_width,
                            int shift_slot, int scale_slot, float eps, void* stream) {
  NormArgs p{};
  p.x = (const uint16_t*)x; p.w = (const uint16_t*)weight; p.table = (const uint16_t*)table;
  p.indices = indices; p.out = (uint16_t*)out;
  p.sequence = sequence; p.hidden = hidden; p.table_rows = table_rows;
  p.table_width = table_width; p.shift_slot = shift_slot; p.scale_slot = scale_slot;
  p.eps = eps;
  if (rows == 0) return LR_OK;
  int rc = check_common(p, rows, max_slot(shift_slot, scale_slot));
  if (rc) return rc;
  LR_REQUIRE(out, "rms_adaln: null output");
  return launch_norm<false, false>(p, rows, vec_ok(p), as_stream(stream));
}

extern "C" int lr_rms_adaln_quant(const void* x, const void* weight, const void* table,
                                  const int64_t* indices, int8_t* q, float* scales, int64_t rows,
                                  int64_t sequence, int64_t hidden, int64_t table_rows,
                                  int64_t table_width, int shift_slot, int scale_slot, float eps,
                                  void* stream) {
  NormArgs p{};
  p.x = (const uint16_t*)x; p.w = (const uint16_t*)weight; p.table = (const uint16_t*)table;
  p.indices = indices; p.q = q; p.scales = scales;
  p.sequence = sequence; p.hidden = hidden; p.table_rows = table_rows;
  p.table_width = table_width; p.shift_slot = shift_slot; p.scale_slot = scale_slot;
  p.eps = eps;
  if (rows == 0) return LR_OK;
  int rc = check_common(p, rows, max_slot(shift_slot, scale_slot));
  if (rc) return rc;
  LR_REQUIRE(q && scales, "rms_adaln_quant: null output");
  return launch_norm<false, true>(p, rows, vec_ok(p), as_stream(stream));
}

extern "C" int lr_residual_rms_quant(const void* x, const void* update, const void* weight,
                                     const void* table, const int64_t* indices,
                                     void* residual_out, int8_t* q, float* scales, int64_t rows,
                                     int64_t sequence, int64_t hidden, int64_t table_rows,
                                     int64_t table_width, float eps, void* stream) {
  NormArgs p{};
  p.x = (const uint16_t*)x; p.u = (const uint16_t*)update; p.w = (const uint16_t*)weight;
  p.table = (const uint16_t*)table; p.indices = indices;
  p.resid_out = (uint16_t*)residual_out; p.q = q; p.scales = scales;
  p.sequence = sequence; p.hidden = hidden; p.table_rows = table_rows;
  p.table_width = table_width; p.shift_slot = 3; p.scale_slot = 4; p.gate_slot = 2;
  p.eps = eps;
  if (rows == 0) return LR_OK;
  int rc = check_common(p, rows, 5);
  if (rc) return rc;
  LR_REQUIRE(update && residual_out && q && scales, "residual_rms_quant: null pointer");
  return launch_norm<true, true>(p, rows, vec_ok(p), as_stream(stream));
}
