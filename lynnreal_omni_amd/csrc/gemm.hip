// gemm.hip - INT8 x INT8 -> INT32 GEMM on CDNA4 MFMA with fused epilogues.
//
// Restates model/int8_gemm.py:13-46 (_gemm) and :84-92 (_torch_matmul):
//   acc[m,n] = sum_k A[m,k] * W[n,k]                        (exact int32)
//   y[m,n]   = bf16(((float)acc * row_scale[m]) * col_scale[n] + bias[n])
// plus GELU-tanh and gated-residual epilogues and a raw-int32 debug output.
//
// Fast kernel (A [M,K] row-major, W [N,K] row-major, K % 16 == 0):
//  * Block tile BM x BN, 4 or 8 waves in a WAVES_M x WAVES_N grid; each wave
//    owns a (BM/WAVES_M) x (BN/WAVES_N) sub-tile of 16x16 MFMA tiles
//    (v_mfma_i32_16x16x64_i8). At most 128 accumulators per wave, held in
//    VGPRs (this file is compiled with -amdgpu-mfma-vgpr-form), so two waves
//    share each SIMD and one wave's waits hide under the other's MFMAs.
//  * Global -> LDS by buffer_load ... lds (16 bytes per lane, no VGPRs), in
//    k-steps of 128 bytes so that each DMA reads whole 128-byte lines; LDS is
//    double-buffered and XOR-swizzled for conflict-free ds_read_b128.
//  * Buffer descriptors bound each block's rows, so rows past M/N and k past
//    K read as zero: no masking in the main loop, tails are exact.
//  * The MFMA is issued as W_frag x A_frag, so lane l ends with row l%16 and
//    4 consecutive columns of C: the epilogue writes 8-byte bf16 groups.
//  * Workgroups are dispatched round-robin over the 8 XCDs; the tile order
//    is renumbered so that each XCD walks a contiguous, M-grouped range of
//    tiles and its 4 MB L2 holds the A and W panels its CUs share.
// Generic kernel: any W strides / K, LDS-tiled int32 dot products (slow path
// used only when the fast kernel cannot run).
#include <mutex>

#include "lr_device.h"
#include "lr_runtime.h"

#ifndef GEMM_RING_A
#define GEMM_RING_A 3
#endif
#ifndef GEMM_RING_B
#define GEMM_RING_B 2
#endif
// Raise the wave's priority for the MFMA stream of each k-step (the two
// waves of a SIMD then issue their MFMAs back to back instead of trading
// issue slots with the other wave's memory instructions): +2% on QKV.
// Ring depth of the 64x128 tile (both operands): its k-steps are small, so
// more of them fit in LDS in flight.
#ifndef GEMM_DEPTH_SMALL
#define GEMM_DEPTH_SMALL 4
#endif
#ifndef GEMM_SETPRIO
#define GEMM_SETPRIO 1
#endif
// Ping-pong k-loop for the 8-wave tiles (K % 128 == 0).
#ifndef GEMM_PINGPONG
#define GEMM_PINGPONG 1
#endif
// Waves (along M) of the 256x80 tile.
#ifndef GEMM_SKINNY_WAVES
#define GEMM_SKINNY_WAVES 4
#endif
// Ring depths (A, W) of the weight-streaming tiles.
#ifndef GEMM_SKINNY_NA
#define GEMM_SKINNY_NA 4
#endif
#ifndef GEMM_SKINNY_NB
#define GEMM_SKINNY_NB 3
#endif
#ifndef GEMM_SKINNY64_NA
#define GEMM_SKINNY64_NA 4
#endif
#ifndef GEMM_SKINNY64_NB
#define GEMM_SKINNY64_NB 4
#endif
#ifndef GEMM_SKINNY128_NA
#define GEMM_SKINNY128_NA 4
#endif
#ifndef GEMM_SKINNY128_NB
#define GEMM_SKINNY128_NB 4
#endif
// Staging rows whose residual and gate chunks the gated epilogue loads
// before using any of them, where it divides the wave's rows of chunks (else
// 4). Chain timings: 6 took FFN-down's 192x256 tiles (12 rows) from 900 to
// 896-897 us; 8 spills registers in the 256x256 tile (out-proj 281 -> 342 us)
// and 12 in the 192x256 one (900 -> 1416 us).
#ifndef GEMM_GATED_BATCH
#define GEMM_GATED_BATCH 6
#endif
// Rows of tiles per raster group of the XCD-aware tile order.
#ifndef GEMM_GROUP_M
#define GEMM_GROUP_M 8
#endif

namespace lr {
namespace {

struct GemmArgs {
  const int8_t* a;
  const int8_t* b;
  const float* rs;
  const float* cs;
  const uint16_t* bias;
  void* c;
  const uint16_t* resid;
  const uint16_t* table;
  const int64_t* indices;
  int64_t m, n, k;
  int64_t b_sk, b_sn;
  int64_t table_rows, table_width, sequence;
  int gate_slot;
  int tiles_m, tiles_n, group_m;
  int splits;  // split-K: workgroups per tile along K (1: none); their int32 partials go to c
  int nvec;    // N % 4 == 0 and C/bias/col_scale/residual aligned for 4-wide access
  int staged;  // nvec, N % 8 == 0 and 16-byte aligned C/residual/table rows: whole-line stores
};

enum { EPI_BF16 = LR_EPI_BF16, EPI_GELU = LR_EPI_GELU_TANH, EPI_GATED = LR_EPI_GATED_RESIDUAL,
       EPI_RAW = LR_EPI_RAW_INT32 };

// ------------------------------------------------------------ epilogue ----
// The bf16 GEMM value, model/int8_gemm.py:42-45 / :89-92 (no FMA contraction).
template <bool BIAS>
__device__ __forceinline__ float dequant(int acc, float rs, float cs, float bias) {
  float v = ((float)acc * rs) * cs;
  if (BIAS) v = v + bias;
  return v;
}

// Final value of one output element for the bf16-producing epilogues.
// gate/x are only read for EPI_GATED.
template <int EPI>
__device__ __forceinline__ float finish(float v, float gate, float x) {
  if (EPI == EPI_GELU) return fast_gelu_tanh(round_bf(v));
  if (EPI == EPI_GATED) return x + round_bf(gate * round_bf(v));
  return v;
}

__device__ __forceinline__ int64_t table_row(const GemmArgs& p, int64_t row) {
  return clamp_index(p.indices[row % p.sequence], p.table_rows);
}

// Stores one element (any shape / alignment).
template <int EPI, bool BIAS>
__device__ __forceinline__ void store_scalar(const GemmArgs& p, int64_t row, int64_t col,
                                             int acc) {
  const int64_t o = row * p.n + col;
  if (EPI == EPI_RAW) {
    static_cast<int32_t*>(p.c)[o] = acc;
    return;
  }
  const float bias = BIAS ? bf_to_f(p.bias[col]) : 0.0f;
  float v = dequant<BIAS>(acc, p.rs[row], p.cs[col], bias);
  float gate = 0.0f, x = 0.0f;
  if (EPI == EPI_GATED) {
    gate = bf_to_f(p.table[table_row(p, row) * p.table_width + (int64_t)p.gate_slot * p.n + col]);
    x = bf_to_f(p.resid[o]);
  }
  v = finish<EPI>(v, gate, x);
  static_cast<uint16_t*>(p.c)[o] = (uint16_t)(pack_bf2(v, 0.0f) & 0xffffu);
}

// ----------------------------------------------------------- tile order ----
// pid is the tile's position in launch order; the hardware deals workgroups
// to the 8 XCDs round-robin, so pid % 8 is the XCD (for a persistent grid
// too, whose size is a multiple of 8).
__device__ __forceinline__ void tile_coords(const GemmArgs& p, int pid, int& tm, int& tn) {
  const int total = p.tiles_m * p.tiles_n;
  const int xcd = pid & 7, local = pid >> 3;
  const int q = total >> 3, r = total & 7;
  const int lid = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
  const int span = p.group_m * p.tiles_n;
  const int g = lid / span;
  const int first = g * p.group_m;
  const int gm = min(p.tiles_m - first, p.group_m);
  const int within = lid - g * span;
  tm = first + within % gm;
  tn = within / gm;
}

// Epilogue of one wave's (16*FM) x (16*FN) sub-tile, stored from the MFMA
// layout: lane l holds, for MFMA tile (i, j), row wm*WM + 16i + l%16 and
// columns wn*WN + 16j + 4*(l/16) + 0..3 (8-byte stores; any N % 4 == 0).
template <int FM, int FN, int WM, int WN, int EPI, bool BIAS>
__device__ __forceinline__ void store_tile(const GemmArgs& p, const v4i (&acc)[FM][FN], int64_t m0,
                                           int64_t n0, int wm, int wn, int lane) {
  const int lr_ = lane & 15, lg = lane >> 4;
  int64_t rows[FM];
  float rsv[FM];
  int64_t trow[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    rows[i] = m0 + wm * WM + 16 * i + lr_;
    const bool ok = rows[i] < p.m;
    rsv[i] = (EPI != EPI_RAW && ok) ? p.rs[rows[i]] : 0.0f;
    trow[i] = (EPI == EPI_GATED && ok) ? table_row(p, rows[i]) : 0;
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    // Keep the column groups apart: hoisting every accumulator read to the
    // top would need all 256 accumulators in VGPRs at once.
    __builtin_amdgcn_sched_barrier(0);
    const int64_t col = n0 + wn * WN + 16 * j + 4 * lg;
    if (p.nvec) {
      if (col >= p.n) continue;
      if (EPI == EPI_RAW) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
          if (rows[i] < p.m)
            store_nt(reinterpret_cast<uint4*>(static_cast<int32_t*>(p.c) + rows[i] * p.n + col),
                     make_uint4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]));
        continue;
      }
      const float4 cs = *reinterpret_cast<const float4*>(p.cs + col);
      float b0 = 0.f, b1 = 0.f, b2 = 0.f, b3 = 0.f;
      if (BIAS) {
        const uint2 bb = *reinterpret_cast<const uint2*>(p.bias + col);
        b0 = bf_lo(bb.x); b1 = bf_hi(bb.x); b2 = bf_lo(bb.y); b3 = bf_hi(bb.y);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if (rows[i] >= p.m) continue;
        const int64_t o = rows[i] * p.n + col;
        float v0 = dequant<BIAS>(acc[i][j][0], rsv[i], cs.x, b0);
        float v1 = dequant<BIAS>(acc[i][j][1], rsv[i], cs.y, b1);
        float v2 = dequant<BIAS>(acc[i][j][2], rsv[i], cs.z, b2);
        float v3 = dequant<BIAS>(acc[i][j][3], rsv[i], cs.w, b3);
        if (EPI == EPI_GATED) {
          const uint2 xv = *reinterpret_cast<const uint2*>(p.resid + o);
          const uint2 gv = *reinterpret_cast<const uint2*>(
              p.table + trow[i] * p.table_width + (int64_t)p.gate_slot * p.n + col);
          v0 = finish<EPI>(v0, bf_lo(gv.x), bf_lo(xv.x));
          v1 = finish<EPI>(v1, bf_hi(gv.x), bf_hi(xv.x));
          v2 = finish<EPI>(v2, bf_lo(gv.y), bf_lo(xv.y));
          v3 = finish<EPI>(v3, bf_hi(gv.y), bf_hi(xv.y));
        } else {
          v0 = finish<EPI>(v0, 0.f, 0.f);
          v1 = finish<EPI>(v1, 0.f, 0.f);
          v2 = finish<EPI>(v2, 0.f, 0.f);
          v3 = finish<EPI>(v3, 0.f, 0.f);
        }
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.c) + o) =
            make_uint2(pack_bf2(v0, v1), pack_bf2(v2, v3));
      }
    } else {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if (rows[i] >= p.m) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (col + e < p.n) store_scalar<EPI, BIAS>(p, rows[i], col + e, acc[i][j][e]);
      }
    }
  }
}

// Whole-line output stores, non-temporal: the output is not read again by
// this kernel, and streaming it keeps the L2 for the operand panels (FFN-up
// 1135 -> 1107 us, the other projections 1-2% faster).
__device__ __forceinline__ void store_c16(uint16_t* dst, const uint4& v) {
  store_nt(reinterpret_cast<uint4*>(dst), v);
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Epilogue through the wave's LDS staging area (row pitch 2*WN + 16 bytes:
// 16-byte aligned rows, and the MFMA-layout writes spread over the banks). Phase 1, in the MFMA layout:
// bf16(((float)acc * rs) * cs + bias) into LDS; for GELU and the gated
// residual this is exactly the bf16 value those epilogues start from. Phase 2,
// row-major: each lane takes 8 consecutive columns of one row (16 bytes),
// finishes the epilogue there (residual and gate read as 16-byte rows) and
// stores them, so that every store instruction writes whole 128-byte lines.
// Partial-line stores from the MFMA layout cost about twice the output bytes
// in HBM writes. Needs N % 8 == 0 and 16-byte aligned C (and residual/table).
template <int FM, int FN, int WM, int WN, int EPI, bool BIAS>
__device__ __forceinline__ void store_tile_staged(const GemmArgs& p, const v4i (&acc)[FM][FN],
                                                  char* stage, int64_t m0, int64_t n0, int wm,
                                                  int wn, int lane) {
  constexpr int PITCH = 2 * WN + 16;
  const int lr_ = lane & 15, lg = lane >> 4;
  // Every scale and bias load of the wave is issued before the first is used
  // (one memory round trip per tile, not one per column group), from clamped
  // addresses so that no load sits under a branch.
  float rsv[FM];
  float4 csv[FN];
  uint2 bv[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t row = m0 + wm * WM + 16 * i + lr_;
    rsv[i] = p.rs[row < p.m ? row : p.m - 1];
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * WN + 16 * j + 4 * lg;
    const int64_t c = col < p.n ? col : p.n - 4;  // N % 8 == 0 on this path
    csv[j] = *reinterpret_cast<const float4*>(p.cs + c);
    if (BIAS) bv[j] = *reinterpret_cast<const uint2*>(p.bias + c);
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    __builtin_amdgcn_sched_barrier(0);
    const float4 cs = csv[j];
    float b0 = 0.f, b1 = 0.f, b2 = 0.f, b3 = 0.f;
    if (BIAS) {
      b0 = bf_lo(bv[j].x); b1 = bf_hi(bv[j].x); b2 = bf_lo(bv[j].y); b3 = bf_hi(bv[j].y);
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const float v0 = dequant<BIAS>(acc[i][j][0], rsv[i], cs.x, b0);
      const float v1 = dequant<BIAS>(acc[i][j][1], rsv[i], cs.y, b1);
      const float v2 = dequant<BIAS>(acc[i][j][2], rsv[i], cs.z, b2);
      const float v3 = dequant<BIAS>(acc[i][j][3], rsv[i], cs.w, b3);
      *reinterpret_cast<uint2*>(stage + (16 * i + lr_) * PITCH + (16 * j + 4 * lg) * 2) =
          make_uint2(pack_bf2(v0, v1), pack_bf2(v2, v3));
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes are done
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);

  constexpr int CPR = WN / 8;                   // 16-byte chunks per row
  constexpr int ITERS = (WM * CPR + 63) / 64;   // rows of 16-byte chunks per lane
  constexpr bool kWhole = WM * CPR % 64 == 0;   // else the last pass is partial
  static_assert(WN % 8 == 0, "staging tile shape");
  const bool seq_covers = p.sequence >= p.m;
  if constexpr (EPI == EPI_GATED && WM <= 128 && kWhole && ITERS % 4 == 0) {
    // x + bf16(gate * y): the residual and gate chunks of 4 staging rows are
    // loaded before any of them is used, from clamped (always valid)
    // addresses, so the loads overlap instead of each waiting in turn (a load
    // under a branch, or after a store the compiler cannot prove disjoint,
    // would serialise them). The table row of each of the wave's WM rows is
    // read once, by lane r % 64 (rows 64.. into a second register), and
    // fetched per chunk with ds_bpermute. The residual is read once
    // (non-temporal loads); the gate rows are shared.
    auto table_row_of = [&](int r) {
      const int64_t row = m0 + wm * WM + (r < WM ? r : 0);
      return (int)clamp_index(
          p.indices[row < p.m ? (seq_covers ? row : row % p.sequence) : 0], p.table_rows);
    };
    const int tr_lane = table_row_of(lane);
    const int tr_lane_hi = WM > 64 ? table_row_of(64 + lane) : 0;
    constexpr int BATCH = ITERS % GEMM_GATED_BATCH == 0 ? GEMM_GATED_BATCH : 4;
#pragma unroll 1
    for (int s0 = 0; s0 < ITERS; s0 += BATCH) {
      uint4 xv[BATCH], gv[BATCH], v[BATCH];
      int64_t o[BATCH];
      bool ok[BATCH];
#pragma unroll
      for (int b = 0; b < BATCH; ++b) {
        const int q = (s0 + b) * 64 + lane;
        const int r = q / CPR, ch = q % CPR;
        const int64_t row = m0 + wm * WM + r;
        const int64_t col = n0 + wn * WN + ch * 8;
        ok[b] = row < p.m && col < p.n;
        const int64_t row_l = ok[b] ? row : m0, col_l = ok[b] ? col : n0;
        o[b] = row * p.n + col;
        const int tr_lo = __builtin_amdgcn_ds_bpermute(4 * r, tr_lane);
        const int tr = WM > 64 ? (r < 64 ? tr_lo : __builtin_amdgcn_ds_bpermute(4 * (r - 64), tr_lane_hi))
                               : tr_lo;
        xv[b] = load_nt(reinterpret_cast<const uint4*>(p.resid + row_l * p.n + col_l));
        gv[b] = *reinterpret_cast<const uint4*>(p.table + (int64_t)tr * p.table_width +
                                                 (int64_t)p.gate_slot * p.n + col_l);
        v[b] = *reinterpret_cast<const uint4*>(stage + r * PITCH + ch * 16);
      }
#pragma unroll
      for (int b = 0; b < BATCH; ++b) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t u = word_of(v[b], w), x = word_of(xv[b], w), g = word_of(gv[b], w);
          const uint32_t y = pack_bf2(bf_lo(x) + round_bf(bf_lo(g) * bf_lo(u)),
                                      bf_hi(x) + round_bf(bf_hi(g) * bf_hi(u)));
          if (w == 0) v[b].x = y; else if (w == 1) v[b].y = y; else if (w == 2) v[b].z = y; else v[b].w = y;
        }
        if (ok[b]) store_c16(static_cast<uint16_t*>(p.c) + o[b], v[b]);
      }
    }
    return;
  }
#pragma unroll 4
  for (int s = 0; s < ITERS; ++s) {
    const int q = s * 64 + lane;
    if (!kWhole && q >= WM * CPR) break;
    const int r = q / CPR, ch = q % CPR;
    const int64_t row = m0 + wm * WM + r;
    const int64_t col = n0 + wn * WN + ch * 8;
    uint4 v = *reinterpret_cast<const uint4*>(stage + r * PITCH + ch * 16);
    if (row < p.m && col < p.n) {
      const int64_t o = row * p.n + col;
      if (EPI == EPI_GELU) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t u = word_of(v, w);
          const uint32_t g = pack_bf2(fast_gelu_tanh(bf_lo(u)), fast_gelu_tanh(bf_hi(u)));
          if (w == 0) v.x = g; else if (w == 1) v.y = g; else if (w == 2) v.z = g; else v.w = g;
        }
      } else if (EPI == EPI_GATED) {
        const int64_t tr = clamp_index(p.indices[seq_covers ? row : row % p.sequence], p.table_rows);
        const uint4 xv = load_nt(reinterpret_cast<const uint4*>(p.resid + o));
        const uint4 gv = *reinterpret_cast<const uint4*>(
            p.table + tr * p.table_width + (int64_t)p.gate_slot * p.n + col);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t u = word_of(v, w), x = word_of(xv, w), g = word_of(gv, w);
          const uint32_t y = pack_bf2(bf_lo(x) + round_bf(bf_lo(g) * bf_lo(u)),
                                      bf_hi(x) + round_bf(bf_hi(g) * bf_hi(u)));
          if (w == 0) v.x = y; else if (w == 1) v.y = y; else if (w == 2) v.z = y; else v.w = y;
        }
      }
      store_c16(static_cast<uint16_t*>(p.c) + o, v);
    }
  }
}

// The raw int32 accumulators through the same per-wave LDS staging area, in
// two column halves (a whole int32 sub-tile is twice the bf16 one; each half
// has the bf16 tile's size and row pitch): every store instruction writes
// whole 128-byte lines. From the MFMA layout each row got 64-byte pieces,
// about 14% more HBM writes than the output. Needs N % 4 == 0 and 16-byte
// aligned C.
template <int FM, int FN, int WM, int WN>
__device__ __forceinline__ void store_tile_staged_raw(const GemmArgs& p, const v4i (&acc)[FM][FN],
                                                      char* stage, int64_t m0, int64_t n0, int wm,
                                                      int wn, int lane) {
  static_assert(FN % 2 == 0, "two column halves");
  constexpr int HALF = FN / 2, HW = WN / 2;
  constexpr int PITCH = 4 * HW + 16;
  constexpr int CPR = HW / 4;            // 16-byte chunks per staging row
  constexpr int ITERS = WM * CPR / 64;
  static_assert(WM * CPR % 64 == 0, "staging tile shape");
  const int lr_ = lane & 15, lg = lane >> 4;
  int32_t* const c = static_cast<int32_t*>(p.c);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int jj = 0; jj < HALF; ++jj)
#pragma unroll
      for (int i = 0; i < FM; ++i)
        *reinterpret_cast<v4i*>(stage + (16 * i + lr_) * PITCH + (16 * jj + 4 * lg) * 4) =
            acc[i][h * HALF + jj];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes are done
    asm volatile("" ::: "memory");
#pragma unroll 4
    for (int s = 0; s < ITERS; ++s) {
      const int q = s * 64 + lane;
      const int r = q / CPR, ch = q % CPR;
      const int64_t row = m0 + wm * WM + r;
      const int64_t col = n0 + wn * WN + h * HW + ch * 4;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + r * PITCH + ch * 16);
      if (row < p.m && col < p.n) store_nt(reinterpret_cast<uint4*>(c + row * p.n + col), v);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // the reads are done before the next half is written
    asm volatile("" ::: "memory");
  }
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from a buffer resource straight into LDS: lane l writes
// lds + 16*l. Offsets past the resource's num_records read as zero.
// (Device-only wrapper: lambdas in kernels are host+device, and the host pass
// must not see the builtin.)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, void* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)lds, 16, voffset, 0, 0, 0);
}
// The same with a wave-uniform byte offset added (an SGPR operand).
__device__ __forceinline__ void dma16s(__amdgpu_buffer_rsrc_t rsrc, void* lds, uint32_t voffset,
                                       uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)lds, 16, voffset, soffset, 0, 0);
}

// ----------------------------------------------------------- fast GEMM ----
// K is consumed in k-steps of 128 bytes; two k-steps live in LDS (double
// buffer). LDS image of one k-step of A (W is the same): 1 KB blocks of 8
// rows x 128 bytes, written by one 16-byte-per-lane DMA each, so every DMA
// reads 8 whole 128-byte lines (a 16-row x 64-byte shape runs the vector
// memory path at a quarter of its rate). Within a row the eight 16-byte
// chunks are stored XOR-swizzled: chunk c of row R sits in slot c ^ (R % 8).
// For the MFMA read (lane l: row l % 16 of a 16-row fragment, chunk l / 16,
// +4 for the second k64 half) each group of 8 lanes then reads 8 distinct
// 16-byte bank groups; measured on gfx950 this runs ds_read_b128 at 94% of
// the rate of a contiguous read (an extra (R / 8) % 2 term drops it to 71%).
//
// Each workgroup computes one tile (gemm_stream is the persistent form).
//
// Split-K (p.splits = S > 1, one tile per workgroup, raw int32 epilogue):
// workgroup g computes k-steps [s * KT / S, (s + 1) * KT / S) of tile g / S,
// s = g % S, and writes those partial sums to slice s of
// p.c (int32 [S, M, N]); splitk_reduce adds the slices (exact integer sums,
// so any split gives the same int32 result) and applies the epilogue.
template <int BM, int BN, int WAVES_M, int WAVES_N, int EPI, bool BIAS, int NA, int NB, bool KALIGNED,
          bool PP>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_fast(GemmArgs p) {
  constexpr int BK = 128;
  constexpr int NWAVES = WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;
  // 1 KB DMA blocks (8 rows x 128 bytes) per k-step, and per wave. Every wave
  // issues the same count (the wait counts assume it); where the blocks do not
  // divide evenly, the surplus loads repeat the last block (same bytes to the
  // same LDS place).
  constexpr int A_BLOCKS = BM / 8, B_BLOCKS = BN / 8;
  constexpr int A_LOADS = (A_BLOCKS + NWAVES - 1) / NWAVES, B_LOADS = (B_BLOCKS + NWAVES - 1) / NWAVES;
  // A k-steps live in a ring of NA LDS slots, W k-steps in a ring of NB: an
  // operand with d slots is fetched d - 1 k-steps ahead.
  static_assert(NWAVES == 4 || NWAVES == 8, "4 or 8 waves");
  static_assert(BM % 16 == 0 && BN % 16 == 0 && FM * 16 * WAVES_M == BM && FN * 16 * WAVES_N == BN &&
                    FM >= 1 && FN >= 1, "tile shape");
  auto a_block = [](int w, int i) { return min(w * A_LOADS + i, A_BLOCKS - 1); };
  auto b_block = [](int w, int j) { return min(w * B_LOADS + j, B_BLOCKS - 1); };
  // The operand rings, reused after the main loop as the epilogue's staging tiles.
  constexpr int RING_BYTES = NA * A_BYTES + NB * B_BYTES;
  constexpr int STAGING_BYTES = NWAVES * WM * (2 * WN + 16);
  __shared__ __attribute__((aligned(1024)))
  char smem[RING_BYTES > STAGING_BYTES ? RING_BYTES : STAGING_BYTES];
  char* const a_ring = smem;
  char* const b_ring = smem + NA * A_BYTES;

  const int kt_all = (int)((p.k + BK - 1) / BK);
  const int splits = p.splits;
  const int slice = (int)blockIdx.x % splits;
  // k-steps [kbase, kend) of the tile; no slice is empty when splits <= KT.
  const int kbase = slice * kt_all / splits, kend = (slice + 1) * kt_all / splits;
  if (splits > 1) p.c = static_cast<int32_t*>(p.c) + (int64_t)slice * p.m * p.n;
  const int pid = (int)blockIdx.x / splits;
  int tm, tn;
  tile_coords(p, pid, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  // Wave-uniform, so that everything derived from it (LDS addresses, M0) stays scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int64_t K = p.k;
  const int KT = kend - kbase;
  // The k-step of K that k-step kt of this workgroup reads; DMAs issued past
  // its last k-step re-read that one.
  auto kpos = [&](int kt) { return kbase + (kt < KT ? kt : KT - 1); };

  const int64_t rows_a = min((int64_t)BM, p.m - m0);
  const int64_t rows_b = min((int64_t)BN, p.n - n0);
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.a + m0 * K), (short)0, (int)(rows_a * K), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.b + n0 * K), (short)0, (int)(rows_b * K), 0x00020000);

  // DMA lane mapping: block kb covers rows 8kb..8kb+7; lane l writes slot
  // l % 8 of row 8kb + l / 8, which holds chunk (l % 8) ^ (l / 8).
  const int drow = lane >> 3;
  const int dchunk = ((lane & 7) ^ drow) * 16;
  uint32_t a_off[A_LOADS], b_off[B_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) a_off[i] = (uint32_t)((a_block(wave, i) * 8 + drow) * K + dchunk);
#pragma unroll
  for (int j = 0; j < B_LOADS; ++j) b_off[j] = (uint32_t)((b_block(wave, j) * 8 + drow) * K + dchunk);

  // With K % 128 == 0 a DMA's per-lane offset is fixed and the k-step goes in
  // the scalar offset (no vector work per DMA). The rings keep issuing past the
  // last k-step so that the wait counts stay fixed; those DMAs re-read the last
  // k-step (every address stays inside the panel, whether or not the hardware
  // bounds check counts the scalar offset) into slots no k-step reads again.
  // With K % 128 != 0 the last k-step is partial: each lane picks an offset
  // past the descriptor (zeros, no memory access) for chunks at or past K, and
  // past the last k-step every lane does.
  auto dma_a = [&](int kt, int i) {
    if constexpr (KALIGNED) {
      dma16s(ra, a_ring + (kt % NA) * A_BYTES + a_block(wave, i) * 1024, a_off[i],
             (uint32_t)(kpos(kt) * BK));
      return;
    }
    const int64_t kbyte = (int64_t)(kbase + kt) * BK;
    dma16(ra, a_ring + (kt % NA) * A_BYTES + a_block(wave, i) * 1024,
          kt < KT && kbyte + dchunk < K ? a_off[i] + (uint32_t)kbyte : 0x80000000u);
  };
  auto dma_b = [&](int kt, int j) {
    if constexpr (KALIGNED) {
      dma16s(rb, b_ring + (kt % NB) * B_BYTES + b_block(wave, j) * 1024, b_off[j],
             (uint32_t)(kpos(kt) * BK));
      return;
    }
    const int64_t kbyte = (int64_t)(kbase + kt) * BK;
    dma16(rb, b_ring + (kt % NB) * B_BYTES + b_block(wave, j) * 1024,
          kt < KT && kbyte + dchunk < K ? b_off[j] + (uint32_t)kbyte : 0x80000000u);
  };
  auto issue_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) dma_a(kt, i);
  };
  auto issue_b = [&](int kt) {
#pragma unroll
    for (int j = 0; j < B_LOADS; ++j) dma_b(kt, j);
  };

  // Fragment read: 16-row fragment f spans blocks 2f, 2f+1.
  const int r16 = lane & 15;
  const int rd_key = r16 & 7;
  const int rd_row = (r16 >> 3) * 1024 + (r16 & 7) * 128;
  const int rd_slot0 = (((lane >> 4) + 0) ^ rd_key) * 16;
  const int rd_slot1 = (((lane >> 4) + 4) ^ rd_key) * 16;
  auto frag = [&](const char* base, int f, int h) -> v4i {
    return *reinterpret_cast<const v4i*>(base + f * 2048 + rd_row + (h ? rd_slot1 : rd_slot0));
  };

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  if constexpr (PP) {
    // Ping-pong: waves 0-3 (one per SIMD) and waves 4-7 (the other wave of each
    // SIMD) alternate between a compute phase (the 64 MFMAs of one k-step, from
    // registers, no other instruction) and a memory phase (the 24 fragment reads
    // of their next k-step, plus DMAs), one phase apart, with a barrier between
    // phases. Each SIMD's MFMA pipe is then fed by one wave at a time that
    // issues nothing else, while its partner's LDS reads and DMAs go to other
    // units. Phase 2k: group 0 reads k-step k, group 1 computes k-step k - 1;
    // phase 2k + 1: group 0 computes k-step k, group 1 reads it.
    //
    // A slot of k-step k is free once group 1 has read it (its lgkmcnt(0)
    // before the barrier that ends phase 2k + 1). Group 0 refills the A ring
    // (3 slots): A(k + 2) in its memory phase of k-step k, into the slot of
    // k-step k - 1, and waits for A(k + 1) at the end of its compute phase of
    // k-step k. Group 1 refills the W ring (2 slots) with W(k + 2), into the
    // slot of k-step k, and waits for W(k + 1) before the barrier that ends its
    // memory phase. Both waits land just before the barrier that ends phase
    // 2k + 1, which publishes k-step k + 1 for group 0's read in phase 2k + 2.
    // A wave's DMAs write the q-th quarter of the tile's W rows (q = wave % 4).
    // With four waves across N (wn = q) no other wave of group 1 reads those
    // rows, so the refill goes out as soon as the wave's own reads are done.
    // With two waves across N each W row is read by two waves of group 1, and
    // one wave's refill could overwrite rows the other is still reading (the
    // per-wave lgkmcnt does not cover other waves): the refill then waits for
    // the barrier that ends phase 2k + 1 and goes out at the start of group
    // 1's compute phase.
    static_assert(NWAVES == 8 && NA == 3 && NB == 2 && KALIGNED, "ping-pong layout");
    constexpr int PA = BM / 8 / 4, PB = BN / 8 / 4;  // 1 KB DMAs per wave per k-step
    static_assert(PA * 32 == BM && PB * 32 == BN && PA <= 15 && PB <= 15, "ping-pong DMA split");
    const int grp = wave >> 2, q = wave & 3;
    uint32_t pa_off[PA], pb_off[PB];
#pragma unroll
    for (int i = 0; i < PA; ++i) pa_off[i] = (uint32_t)(((q * PA + i) * 8 + drow) * K + dchunk);
#pragma unroll
    for (int j = 0; j < PB; ++j) pb_off[j] = (uint32_t)(((q * PB + j) * 8 + drow) * K + dchunk);
    // DMAs past the last k-step re-read the last one (every address stays in
    // the panel) into slots that no k-step reads again.
    auto pdma_a = [&](int kt) {
      const uint32_t soff = (uint32_t)(kpos(kt) * BK);
#pragma unroll
      for (int i = 0; i < PA; ++i)
        dma16s(ra, a_ring + (kt % NA) * A_BYTES + (q * PA + i) * 1024, pa_off[i], soff);
    };
    auto pdma_b = [&](int kt) {
      const uint32_t soff = (uint32_t)(kpos(kt) * BK);
#pragma unroll
      for (int j = 0; j < PB; ++j)
        dma16s(rb, b_ring + (kt % NB) * B_BYTES + (q * PB + j) * 1024, pb_off[j], soff);
    };
    constexpr int kWaitA = 0x70 | 0xf00 | PA;  // vmcnt(PA): all but the newest k-step landed
    constexpr int kWaitB = 0x70 | 0xf00 | PB;
    constexpr int kWaitLds = 0xc07f;           // lgkmcnt(0)
    constexpr int kWaitLdsVm0 = 0x70;          // vmcnt(0) lgkmcnt(0)
    constexpr bool kOwnW = WAVES_N == 4;       // wn == wave % 4 for every wave
    v4i a0[FM], w0[FN], a1[FM], w1[FN];
    auto read_all = [&](int kt) {
      const char* sa = a_ring + (kt % NA) * A_BYTES;
      const char* sb = b_ring + (kt % NB) * B_BYTES;
#pragma unroll
      for (int i = 0; i < FM; ++i) a0[i] = frag(sa, wm * FM + i, 0);
#pragma unroll
      for (int j = 0; j < FN; ++j) w0[j] = frag(sb, wn * FN + j, 0);
#pragma unroll
      for (int i = 0; i < FM; ++i) a1[i] = frag(sa, wm * FM + i, 1);
#pragma unroll
      for (int j = 0; j < FN; ++j) w1[j] = frag(sb, wn * FN + j, 1);
    };
    auto compute = [&]() {
#pragma unroll
      for (int t = 0; t < FM * FN; ++t) {
        const int i = t / FN, j = t % FN;
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w0[j], a0[i], acc[i][j], 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < FM * FN; ++t) {
        const int i = t / FN, j = t % FN;
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w1[j], a1[i], acc[i][j], 0, 0, 0);
      }
    };
    // The MFMAs touch no memory: without the leading scheduling barrier the
    // compiler would move the s_barrier above them.
    auto barrier = [&]() {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    };
    if (grp == 0) {
      pdma_a(0);
      pdma_a(1);
      __builtin_amdgcn_s_waitcnt(kWaitA);
      barrier();
      for (int kt = 0; kt < KT; ++kt) {
        read_all(kt);  // phase 2kt
        pdma_a(kt + 2);
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        barrier();
        compute();  // phase 2kt + 1
        __builtin_amdgcn_sched_barrier(0);  // the wait stays behind the MFMAs
        __builtin_amdgcn_s_waitcnt(kWaitA);
        barrier();
      }
      barrier();  // phase 2KT: group 1 computes the last k-step
    } else {
      pdma_b(0);
      pdma_b(1);
      __builtin_amdgcn_s_waitcnt(kWaitB);
      barrier();
      barrier();  // phase 0: group 0 reads k-step 0
      for (int kt = 0; kt < KT; ++kt) {
        read_all(kt);  // phase 2kt + 1
        if constexpr (kOwnW) {
          // This wave alone in its group reads the W rows it refills.
          __builtin_amdgcn_s_waitcnt(kWaitLds);
          pdma_b(kt + 2);
          __builtin_amdgcn_s_waitcnt(kWaitB);  // W(kt + 1) landed
          barrier();
        } else {
          // Other waves of this group may still be reading the rows this
          // wave's DMAs would overwrite: refill after the barrier, by which
          // every wave has read W(kt). W(kt + 1), issued one phase ago, is
          // the only load in flight.
          __builtin_amdgcn_s_waitcnt(kWaitLdsVm0);
          barrier();
          pdma_b(kt + 2);
        }
        compute();  // phase 2kt + 2
        barrier();
      }
    }
  } else {
  // One barrier per k-step, between its two halves. Fragments are always read
  // one half ahead: the second half's while the first half's MFMAs run, and the
  // next k-step's first half while the second half's MFMAs run, so no MFMA
  // waits for an LDS read issued after a barrier. At the barrier in k-step kt
  // every wave has its k-step kt fragments in registers (lgkmcnt(0)), so the
  // slots of k-step kt are free: the second half refills them with k-step
  // kt + NA (A) and kt + NB (W), i.e. each ring keeps all of its slots in
  // flight. The barrier also publishes k-step kt + 1, whose DMAs each wave
  // has waited for (vmcnt) just before it.
  //
  // DMA issue order per wave: round t issues W(t + NB) then A(t + NA) (rounds
  // -max(NA, NB) .. -1 form the prologue, round t >= 0 is the second half of
  // k-step t; indices below 0 are skipped). Loads still allowed in flight:
  //   before k-step 0 (A(0), W(0) landed):     kPro
  //   at the barrier of k-step kt (A(kt+1), W(kt+1) landed): kMid
  static_assert(NA >= 2 && NB >= 2, "ring depths");
  constexpr int kStep = A_LOADS + B_LOADS;
  constexpr int kPro = NA > NB ? A_LOADS + (NB - 1) * kStep : (NA - 1) * kStep;
  constexpr int kMid = NA > NB ? A_LOADS + (NB - 2) * kStep : (NA - 2) * kStep;
  static_assert(kPro <= 63 && kMid >= 0, "vmcnt range");
  constexpr int kWaitPro = 0x70 | 0xf00 | (kPro & 0xf) | ((kPro >> 4) << 14);  // vmcnt(kPro)
  constexpr int kWaitMid = 0x70 | (kMid & 0xf) | ((kMid >> 4) << 14);  // vmcnt(kMid) lgkmcnt(0)
  constexpr int NMAX = NA > NB ? NA : NB;
#pragma unroll
  for (int t = -NMAX; t < 0; ++t) {
    if (t + NB >= 0) issue_b(t + NB);
    if (t + NA >= 0) issue_a(t + NA);
  }
  constexpr int NMF = FM * FN;
  constexpr int NR = FM + FN;
  constexpr int ND = A_LOADS + B_LOADS;
  v4i a0[FM], w0[FN], a1[FM], w1[FN];
  // Fragment r of a half in MFMA order: a[0], w[0..FN-1], a[1..FM-1] (the
  // first MFMA needs two reads, each later one at most one new read).
  auto read_half = [&](const char* sa, const char* sb, int h, int r, v4i (&av)[FM], v4i (&wv)[FN]) {
    if (r == 0) av[0] = frag(sa, wm * FM, h);
    else if (r <= FN) wv[r - 1] = frag(sb, wn * FN + r - 1, h);
    else av[r - FN] = frag(sa, wm * FM + r - FN, h);
  };
  __builtin_amdgcn_s_waitcnt(kWaitPro);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < NR; ++r) read_half(a_ring, b_ring, 0, r, a0, w0);
  __builtin_amdgcn_sched_barrier(0);

  for (int kt = 0; kt < KT; ++kt) {
    const char* sa = a_ring + (kt % NA) * A_BYTES;
    const char* sb = b_ring + (kt % NB) * B_BYTES;
    const char* na = a_ring + ((kt + 1) % NA) * A_BYTES;
    const char* nb = b_ring + ((kt + 1) % NB) * B_BYTES;
#if GEMM_SETPRIO
    __builtin_amdgcn_s_setprio(1);
#endif
    // First half: MFMAs on (a0, w0); this k-step's second-half fragments read.
#pragma unroll
    for (int t = 0; t < NMF; ++t) {
      const int i = t / FN, j = t % FN;
      acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w0[j], a0[i], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int r = 0; r < NR; ++r)
        if ((r * NMF) / NR == t) read_half(sa, sb, 1, r, a1, w1);
      __builtin_amdgcn_sched_barrier(0);
    }
#if GEMM_SETPRIO
    __builtin_amdgcn_s_setprio(0);
#endif
    __builtin_amdgcn_s_waitcnt(kWaitMid);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#if GEMM_SETPRIO
    __builtin_amdgcn_s_setprio(1);
#endif
    // Second half: MFMAs on (a1, w1); the next k-step's first-half fragments
    // read; this k-step's slots refilled (W first, then A).
#pragma unroll
    for (int t = 0; t < NMF; ++t) {
      const int i = t / FN, j = t % FN;
      acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w1[j], a1[i], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int r = 0; r < NR; ++r)
        if ((r * NMF) / NR == t) read_half(na, nb, 0, r, a0, w0);
#pragma unroll
      for (int d = 0; d < ND; ++d) {
        if ((d * NMF) / ND == t) {
          if (d < B_LOADS) dma_b(kt + NB, d);
          else dma_a(kt + NA, d - B_LOADS);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#if GEMM_SETPRIO
    __builtin_amdgcn_s_setprio(0);
#endif
  }
  }
  // The trailing zero-fill DMAs must land before the workgroup's LDS is freed.
  __builtin_amdgcn_s_waitcnt(0x70 | 0xf00);  // vmcnt(0)

  if (EPI != EPI_RAW && p.staged) {
    // Whole-line stores through LDS: every wave must be done reading the
    // operand stages before they are overwritten.
    static_assert(NWAVES * WM * (2 * WN + 16) <= (int)sizeof(smem), "staging fits in LDS");
    __syncthreads();
    store_tile_staged<FM, FN, WM, WN, EPI, BIAS>(p, acc, smem + wave * WM * (2 * WN + 16), m0, n0,
                                                 wm, wn, lane);
  } else if (EPI == EPI_RAW && FN % 2 == 0 && p.nvec) {
    __syncthreads();
    if constexpr (FN % 2 == 0)
      store_tile_staged_raw<FM, FN, WM, WN>(p, acc, smem + wave * WM * (2 * WN + 16), m0, n0, wm,
                                            wn, lane);
  } else {
    store_tile<FM, FN, WM, WN, EPI, BIAS>(p, acc, m0, n0, wm, wn, lane);
  }
}

// ------------------------------------- persistent 256x256, streamed tiles ----
// The persistent form of the 256x256 GEMM behind int8_tma.matmul: a grid of
// at most one workgroup per CU loops over the tiles in launch order (pid =
// blockIdx.x, + gridDim.x, ...), the schedule of the reference's persistent
// kernel (model/int8_tma.py:12-29), with gemm_fast's ping-pong k-loop (2x4
// wave grid). Its tiles follow each other without a cold start: the
// two DMAs that a tile's last k-steps issue past its end, which the
// one-tile-per-workgroup kernel spends re-reading its last k-step, load the
// next tile's k-steps 0 and 1 instead, so the next tile's operands arrive
// while this tile's outputs are written. The ring slots continue across
// tiles (k-step g of the workgroup, counted over its tiles, lives in A slot
// g % 3 and W slot g % 2). The epilogue then has only the A slot of the
// tile's last k-step free (32 KB, 4 KB per wave), so it stages the 128x64
// bf16 outputs of a wave in four passes of 32 rows (row pitch 128 bytes,
// 16-byte chunks XOR-swizzled by row) instead of the whole tile at once.
// K % 128 == 0 and K >= 256.

// The pass-staged epilogue of one wave's 128x64 sub-tile (N % 8 == 0,
// N <= 2^21 and 16-byte aligned outputs): pass p stages rows 32p .. 32p + 31
// (fragments 2p and 2p + 1) in the MFMA layout, then each lane finishes and
// stores 4 whole 16-byte chunks of them.
//
// Scales, bias and outputs go through buffer ranges that start at the tile's
// first row and column and end at M and N: loads past them return zero and
// stores past them are dropped, so no load or store needs a per-row check or a
// 64-bit address. A lane whose columns lie past N stores at byte offset 2^31
// and up, beyond every range (a tile's output range is under 2^30 bytes).
template <int EPI, bool BIAS>
__device__ __forceinline__ void store_tile_passes(const GemmArgs& p, const v4i (&acc)[8][4], char* stage,
                                                  int64_t m0, int64_t n0, int wm, int wn, int lane) {
  constexpr int FM = 8, FN = 4, WM = 128, WN = 64;
  const int lr_ = lane & 15, lg = lane >> 4;
  const int64_t tile_rows = min((int64_t)256, p.m - m0), tile_cols = min((int64_t)256, p.n - n0);
  const __amdgpu_buffer_rsrc_t r_rs = row_rsrc(p.rs + m0, tile_rows * 4);
  const __amdgpu_buffer_rsrc_t r_cs = row_rsrc(p.cs + n0, tile_cols * 4);
  float rsv[FM];
  float4 csv[FN];
  uint2 bv[FN];
  const uint32_t rs_off = (uint32_t)(wm * WM + lr_) * 4;
#pragma unroll
  for (int i = 0; i < FM; ++i)
    rsv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r_rs, rs_off + 64 * i, 0, 0));
  const uint32_t cs_off = (uint32_t)(wn * WN + 4 * lg) * 4;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const v4u c = __builtin_amdgcn_raw_buffer_load_b128(r_cs, cs_off + 64 * j, 0, 0);
    csv[j] = make_float4(__uint_as_float(c.x), __uint_as_float(c.y), __uint_as_float(c.z),
                         __uint_as_float(c.w));
  }
  if (BIAS) {
    const __amdgpu_buffer_rsrc_t r_b = row_rsrc(p.bias + n0, tile_cols * 2);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const v2u b = __builtin_amdgcn_raw_buffer_load_b64(r_b, cs_off / 2 + 32 * j, 0, 0);
      bv[j] = make_uint2(b.x, b.y);
    }
  }
  // Output offsets (non-gated): lane l stores the 16-byte chunk l % 8 of row
  // l / 8 of each group of 8 rows.
  const __amdgpu_buffer_rsrc_t r_c =
      row_rsrc(static_cast<const uint16_t*>(p.c) + m0 * p.n, tile_rows * p.n * 2);
  const int64_t out_col = n0 + wn * WN + (lane & 7) * 8;
  const uint32_t c_off = out_col < p.n ? (uint32_t)(((wm * WM + (lane >> 3)) * p.n + out_col) * 2)
                                       : 0x80000000u;
  const uint32_t rows8 = (uint32_t)(16 * p.n);  // bytes of 8 output rows
  // Everything issued before these loads, the next tile's first operand DMAs
  // among them, has landed once they have (gemm_stream's k-loop relies on it).
  __builtin_amdgcn_s_waitcnt(0x70 | 0xf00);  // vmcnt(0)
  const bool seq_covers = p.sequence >= p.m;
  // Unrolled: the accumulator indices must be constants, or the array would
  // live in scratch memory.
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      float b0 = 0.f, b1 = 0.f, b2 = 0.f, b3 = 0.f;
      if (BIAS) {
        b0 = bf_lo(bv[j].x); b1 = bf_hi(bv[j].x); b2 = bf_lo(bv[j].y); b3 = bf_hi(bv[j].y);
      }
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const int i = 2 * pass + ii;
        const float v0 = dequant<BIAS>(acc[i][j][0], rsv[i], csv[j].x, b0);
        const float v1 = dequant<BIAS>(acc[i][j][1], rsv[i], csv[j].y, b1);
        const float v2 = dequant<BIAS>(acc[i][j][2], rsv[i], csv[j].z, b2);
        const float v3 = dequant<BIAS>(acc[i][j][3], rsv[i], csv[j].w, b3);
        const int r = 16 * ii + lr_;
        const int chunk = (2 * j + (lg >> 1)) ^ (r & 7);
        *reinterpret_cast<uint2*>(stage + r * 128 + chunk * 16 + (lg & 1) * 8) =
            make_uint2(pack_bf2(v0, v1), pack_bf2(v2, v3));
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes are done
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // Gated: two chunks at a time (their residual and gate loads in flight
    // together); four at once spill registers next to the accumulators.
    constexpr int BATCH = EPI == EPI_GATED ? 2 : 4;
#pragma unroll
    for (int s0 = 0; s0 < 4; s0 += BATCH) {
      uint4 v[BATCH], xv[BATCH], gv[BATCH];
      int64_t o[BATCH];
      bool ok[BATCH];
#pragma unroll
      for (int b = 0; b < BATCH; ++b) {
        const int q = (s0 + b) * 64 + lane;
        const int r = q >> 3, ch = q & 7;
        v[b] = *reinterpret_cast<const uint4*>(stage + r * 128 + ((ch ^ (r & 7)) << 4));
        if (EPI == EPI_GATED) {
          const int64_t row = m0 + wm * WM + 32 * pass + r;
          const int64_t col = n0 + wn * WN + ch * 8;
          ok[b] = row < p.m && col < p.n;
          o[b] = row * p.n + col;
          // Clamped (always valid) addresses, so that no load sits under a branch.
          const int64_t row_l = ok[b] ? row : m0, col_l = ok[b] ? col : n0;
          const int64_t tr = clamp_index(
              p.indices[row < p.m ? (seq_covers ? row : row % p.sequence) : 0], p.table_rows);
          xv[b] = load_nt(reinterpret_cast<const uint4*>(p.resid + row_l * p.n + col_l));
          gv[b] = *reinterpret_cast<const uint4*>(p.table + tr * p.table_width +
                                                   (int64_t)p.gate_slot * p.n + col_l);
        }
      }
#pragma unroll
      for (int b = 0; b < BATCH; ++b) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t u = word_of(v[b], w);
          uint32_t y = u;
          if (EPI == EPI_GELU) {
            y = pack_bf2(fast_gelu_tanh(bf_lo(u)), fast_gelu_tanh(bf_hi(u)));
          } else if (EPI == EPI_GATED) {
            const uint32_t x = word_of(xv[b], w), g = word_of(gv[b], w);
            y = pack_bf2(bf_lo(x) + round_bf(bf_lo(g) * bf_lo(u)), bf_hi(x) + round_bf(bf_hi(g) * bf_hi(u)));
          }
          if (w == 0) v[b].x = y; else if (w == 1) v[b].y = y; else if (w == 2) v[b].z = y; else v[b].w = y;
        }
        if (EPI == EPI_GATED) {
          if (ok[b]) store_c16(static_cast<uint16_t*>(p.c) + o[b], v[b]);
        } else {
          const v4u w = {v[b].x, v[b].y, v[b].z, v[b].w};
          __builtin_amdgcn_raw_buffer_store_b128(w, r_c, c_off + (uint32_t)(4 * pass + s0 + b) * rows8, 0,
                                                 2 /* nt */);
        }
      }
    }
    // This pass's chunks are in registers before the next pass overwrites them.
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int EPI, bool BIAS, bool STAGED>
__global__ __launch_bounds__(512) void gemm_stream(GemmArgs p) {
  constexpr int BM = 256, BN = 256, BK = 128, NA = 3, NB = 2, WAVES_N = 4;
  constexpr int WM = 128, WN = 64, FM = 8, FN = 4;
  constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;
  constexpr int PA = 8, PB = 8;  // 1 KB DMAs per wave per k-step
  __shared__ __attribute__((aligned(1024))) char smem[NA * A_BYTES + NB * B_BYTES];
  char* const a_ring = smem;
  char* const b_ring = smem + NA * A_BYTES;

  const int tiles = p.tiles_m * p.tiles_n;
  const int64_t K = p.k;
  const int KT = (int)(K / BK);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int grp = wave >> 2, q = wave & 3;
  const int drow = lane >> 3;
  const int dchunk = ((lane & 7) ^ drow) * 16;
  uint32_t pa_off[PA], pb_off[PB];
#pragma unroll
  for (int i = 0; i < PA; ++i) pa_off[i] = (uint32_t)(((q * PA + i) * 8 + drow) * K + dchunk);
#pragma unroll
  for (int j = 0; j < PB; ++j) pb_off[j] = (uint32_t)(((q * PB + j) * 8 + drow) * K + dchunk);
  const int r16 = lane & 15;
  const int rd_key = r16 & 7;
  const int rd_row = (r16 >> 3) * 1024 + (r16 & 7) * 128;
  const int rd_slot0 = (((lane >> 4) + 0) ^ rd_key) * 16;
  const int rd_slot1 = (((lane >> 4) + 4) ^ rd_key) * 16;
  auto frag = [&](const char* base, int f, int h) -> v4i {
    return *reinterpret_cast<const v4i*>(base + f * 2048 + rd_row + (h ? rd_slot1 : rd_slot0));
  };
  // Panel descriptors of tile pid (rows past M / N read as zero).
  auto panel_a = [&](int pid) {
    int tm, tn;
    tile_coords(p, pid, tm, tn);
    const int64_t m0 = (int64_t)tm * BM;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(p.a + m0 * K), (short)0,
                                             (int)(min((int64_t)BM, p.m - m0) * K), 0x00020000);
  };
  auto panel_b = [&](int pid) {
    int tm, tn;
    tile_coords(p, pid, tm, tn);
    const int64_t n0 = (int64_t)tn * BN;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(p.b + n0 * K), (short)0,
                                             (int)(min((int64_t)BN, p.n - n0) * K), 0x00020000);
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  constexpr int kWaitA = 0x70 | 0xf00 | PA;  // vmcnt(PA): all but the newest k-step landed
  constexpr int kWaitB = 0x70 | 0xf00 | PB;
  constexpr int kWaitLds = 0xc07f;           // lgkmcnt(0)
  // With the staged epilogue, k-step 1 of every tile has landed before its
  // k-loop starts: the first tile's prologue waits for both of its k-steps,
  // and each epilogue waits for its scale loads, issued after the DMAs of the
  // next tile's k-steps 0 and 1 (vmcnt counts in issue order). The loop then
  // skips the wait after k-step 0, the only one that the previous tile's
  // output stores (issued after those DMAs) would otherwise hold up: they
  // drain under the MFMAs of k-steps 0 and 1, and the wait for k-step 2,
  // whose DMAs were issued after them, is the first to cover them.
  constexpr int kWaitAll = 0x70 | 0xf00;  // vmcnt(0)
  static_assert(PA == 8 && PB == 8, "wait_after_first_kstep waits for vmcnt(8)");
  // vmcnt(8) except after k-step 0, as one asm statement: a branch in C++
  // made the compiler peel k-step 0 out of the loop and spill registers.
  auto wait_after_first_kstep = [](int kt) {
    asm volatile("s_cmp_eq_u32 %0, 0\n\ts_cbranch_scc1 1f\n\ts_waitcnt vmcnt(8)\n1:" ::"s"(kt) : "scc");
  };

  int g = 0;  // the workgroup's k-steps before this tile (ring position)
  for (int pid = blockIdx.x; pid < tiles; pid += gridDim.x, g += KT) {
    int tm, tn;
    tile_coords(p, pid, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const bool first = pid == (int)blockIdx.x;
    const int next = pid + (int)gridDim.x;
    const bool has_next = next < tiles;
    const __amdgpu_buffer_rsrc_t ra = panel_a(pid), rb = panel_b(pid);
    const __amdgpu_buffer_rsrc_t ra_n = has_next ? panel_a(next) : ra;
    const __amdgpu_buffer_rsrc_t rb_n = has_next ? panel_b(next) : rb;
    // k-step kt >= KT of this tile is k-step kt - KT of the next one, or past
    // the last tile a re-read of this tile's last k-step.
    auto pdma_a = [&](int kt) {
      const bool nxt = kt >= KT && has_next;
      const uint32_t soff = (uint32_t)((kt < KT ? kt : (nxt ? kt - KT : KT - 1)) * BK);
      char* slot = a_ring + ((g + kt) % NA) * A_BYTES;
#pragma unroll
      for (int i = 0; i < PA; ++i) dma16s(nxt ? ra_n : ra, slot + (q * PA + i) * 1024, pa_off[i], soff);
    };
    auto pdma_b = [&](int kt) {
      const bool nxt = kt >= KT && has_next;
      const uint32_t soff = (uint32_t)((kt < KT ? kt : (nxt ? kt - KT : KT - 1)) * BK);
      char* slot = b_ring + ((g + kt) % NB) * B_BYTES;
#pragma unroll
      for (int j = 0; j < PB; ++j) dma16s(nxt ? rb_n : rb, slot + (q * PB + j) * 1024, pb_off[j], soff);
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    v4i a0[FM], w0[FN], a1[FM], w1[FN];
    auto read_all = [&](int kt) {
      const char* sa = a_ring + ((g + kt) % NA) * A_BYTES;
      const char* sb = b_ring + ((g + kt) % NB) * B_BYTES;
#pragma unroll
      for (int i = 0; i < FM; ++i) a0[i] = frag(sa, wm * FM + i, 0);
#pragma unroll
      for (int j = 0; j < FN; ++j) w0[j] = frag(sb, wn * FN + j, 0);
#pragma unroll
      for (int i = 0; i < FM; ++i) a1[i] = frag(sa, wm * FM + i, 1);
#pragma unroll
      for (int j = 0; j < FN; ++j) w1[j] = frag(sb, wn * FN + j, 1);
    };
    auto compute = [&]() {
#pragma unroll
      for (int t = 0; t < FM * FN; ++t) {
        const int i = t / FN, j = t % FN;
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w0[j], a0[i], acc[i][j], 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < FM * FN; ++t) {
        const int i = t / FN, j = t % FN;
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w1[j], a1[i], acc[i][j], 0, 0, 0);
      }
    };
    // The schedule of gemm_fast's ping-pong loop. A later tile's k-steps 0
    // and 1 were issued by the tile before it, whose last waits (A(KT) and
    // W(KT)) covered k-step 0; with the staged epilogue k-step 1 has landed
    // too, and the loop skips its wait after k-step 0 (kWaitAll above).
    if (grp == 0) {
      if (first) {
        pdma_a(0);
        pdma_a(1);
        __builtin_amdgcn_s_waitcnt(STAGED ? kWaitAll : kWaitA);
      }
      barrier();
      for (int kt = 0; kt < KT; ++kt) {
        read_all(kt);  // phase 2kt
        pdma_a(kt + 2);
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        barrier();
        compute();  // phase 2kt + 1
        __builtin_amdgcn_sched_barrier(0);
        if (STAGED)
          wait_after_first_kstep(kt);
        else
          __builtin_amdgcn_s_waitcnt(kWaitA);
        barrier();
      }
      barrier();  // phase 2KT: group 1 computes the last k-step
    } else {
      if (first) {
        pdma_b(0);
        pdma_b(1);
        __builtin_amdgcn_s_waitcnt(STAGED ? kWaitAll : kWaitB);
      }
      barrier();
      barrier();  // phase 0: group 0 reads k-step 0
      for (int kt = 0; kt < KT; ++kt) {
        read_all(kt);  // phase 2kt + 1
        // With four waves across N this wave alone in its group reads the W
        // rows it refills.
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        pdma_b(kt + 2);
        if (STAGED)  // W(kt + 1) landed
          wait_after_first_kstep(kt);
        else
          __builtin_amdgcn_s_waitcnt(kWaitB);
        barrier();
        compute();  // phase 2kt + 2
        barrier();
      }
    }
    // Every wave has read k-step KT - 1, so its A slot is free for the
    // epilogue; the slots of the next tile's k-steps 0 and 1 stay untouched.
    // The next tile's first barrier keeps its A(2) DMA, which refills this
    // slot, behind every wave's epilogue.
    // One epilogue per instantiation: a loop whose body held both would merge
    // their pending loads at the loop head, and the compiler would then wait
    // for every outstanding memory operation (vmcnt(0)), the output stores
    // included, before the next tile's accumulators are cleared.
    if constexpr (STAGED) {
      char* const stage = a_ring + ((g + KT - 1) % NA) * A_BYTES + wave * 4096;
      store_tile_passes<EPI, BIAS>(p, acc, stage, m0, n0, wm, wn, lane);
    } else {
      store_tile<FM, FN, WM, WN, EPI, BIAS>(p, acc, m0, n0, wm, wn, lane);
    }
  }
  // The last tile's trailing DMAs land before the workgroup's LDS is freed.
  __builtin_amdgcn_s_waitcnt(0x70 | 0xf00);  // vmcnt(0)
}

// -------------------------------------------------------- generic GEMM ----
// 64x64 tile per block, 4x4 outputs per thread, K in steps of 32 through LDS.
template <int EPI, bool BIAS>
__global__ __launch_bounds__(256) void gemm_generic(GemmArgs p) {
  __shared__ int As[32][64 + 1];
  __shared__ int Bs[32][64 + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  int acc[4][4] = {};
  for (int64_t k0 = 0; k0 < p.k; k0 += 32) {
    for (int idx = threadIdx.x; idx < 64 * 32; idx += 256) {
      const int r = idx >> 5, kk = idx & 31;
      const int64_t gm = m0 + r, gk = k0 + kk;
      As[kk][r] = (gm < p.m && gk < p.k) ? (int)p.a[gm * p.k + gk] : 0;
      const int64_t gn = n0 + r;
      Bs[kk][r] = (gn < p.n && gk < p.k) ? (int)p.b[gk * p.b_sk + gn * p.b_sn] : 0;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < 32; ++kk) {
      int av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t row = m0 + ty * 4 + i, col = n0 + tx * 4 + j;
      if (row < p.m && col < p.n) store_scalar<EPI, BIAS>(p, row, col, acc[i][j]);
    }
}

// ---------------------------------------------------- split-K reduce ----
// out[m, n] = epilogue(sum_s part[s, m, n]): the slices of a split-K GEMM
// added in int32 (exact), then the same dequant and epilogue arithmetic as
// the one-pass kernels. With p.staged each thread finishes 8 consecutive
// outputs of one row (32-byte partial loads per slice, one 16-byte store);
// otherwise one output per thread.
template <int EPI, bool BIAS>
__global__ __launch_bounds__(256) void splitk_reduce(GemmArgs p, const int32_t* __restrict__ part,
                                                     int splits) {
  const int64_t mn = p.m * p.n;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (!p.staged) {
    if (t >= mn) return;
    int acc = 0;
    for (int sl = 0; sl < splits; ++sl) acc += part[sl * mn + t];
    store_scalar<EPI, BIAS>(p, t / p.n, t % p.n, acc);
    return;
  }
  const int64_t per_row = p.n / 8;
  if (t >= p.m * per_row) return;
  const int64_t row = t / per_row, col = (t - row * per_row) * 8;
  const int64_t o = row * p.n + col;
  int acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int sl = 0; sl < splits; ++sl) {
    const uint4* src = reinterpret_cast<const uint4*>(part + sl * mn + o);
    const uint4 lo = load_nt(src), hi = load_nt(src + 1);
    acc[0] += (int)lo.x; acc[1] += (int)lo.y; acc[2] += (int)lo.z; acc[3] += (int)lo.w;
    acc[4] += (int)hi.x; acc[5] += (int)hi.y; acc[6] += (int)hi.z; acc[7] += (int)hi.w;
  }
  if (EPI == EPI_RAW) {
    uint4* dst = reinterpret_cast<uint4*>(static_cast<int32_t*>(p.c) + o);
    store_nt(dst, make_uint4(acc[0], acc[1], acc[2], acc[3]));
    store_nt(dst + 1, make_uint4(acc[4], acc[5], acc[6], acc[7]));
    return;
  }
  const float rs = p.rs[row];
  const float4 c0 = *reinterpret_cast<const float4*>(p.cs + col);
  const float4 c1 = *reinterpret_cast<const float4*>(p.cs + col + 4);
  const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  float bias[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (BIAS) unpack8(*reinterpret_cast<const uint4*>(p.bias + col), bias);
  float gate[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (EPI == EPI_GATED) {
    const int64_t tr = table_row(p, row);
    unpack8(*reinterpret_cast<const uint4*>(p.table + tr * p.table_width + (int64_t)p.gate_slot * p.n + col),
            gate);
    unpack8(load_nt(reinterpret_cast<const uint4*>(p.resid + o)), x);
  }
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = finish<EPI>(dequant<BIAS>(acc[e], rs, cs[e], bias[e]), gate[e], x[e]);
  store_c16(static_cast<uint16_t*>(p.c) + o, pack8(v));
}

// ------------------------------------------------------------- launch ----
struct FastCfg {
  int bm, bn;
};

template <int BM, int BN, int WAVES_M, int WAVES_N, int EPI, bool BIAS, int NA = GEMM_RING_A,
          int NB = GEMM_RING_B>
void launch_fast_cfg(GemmArgs& p, hipStream_t st) {
  p.tiles_m = (int)((p.m + BM - 1) / BM);
  p.tiles_n = (int)((p.n + BN - 1) / BN);
  const unsigned grid = (unsigned)(p.tiles_m * p.tiles_n * p.splits);
  constexpr bool kPingPong = GEMM_PINGPONG && WAVES_M * WAVES_N == 8 && NA == 3 && NB == 2;
  if (p.k % 128 == 0)
    hipLaunchKernelGGL((gemm_fast<BM, BN, WAVES_M, WAVES_N, EPI, BIAS, NA, NB, true, kPingPong>),
                       dim3(grid), dim3(64 * WAVES_M * WAVES_N), 0, st, p);
  else
    hipLaunchKernelGGL((gemm_fast<BM, BN, WAVES_M, WAVES_N, EPI, BIAS, NA, NB, false, false>),
                       dim3(grid), dim3(64 * WAVES_M * WAVES_N), 0, st, p);
}

// The persistent 256x256 block, streamed (K % 128 == 0 and K >= 256, else one
// tile per workgroup): one workgroup per CU, rounded down to a multiple of the
// 8 XCDs (so blockIdx % 8 is the XCD, as the tile order assumes).
template <int EPI, bool BIAS>
void launch_persistent(GemmArgs& p, hipStream_t st) {
  if (p.k % 128 != 0 || p.k < 256) {
    launch_fast_cfg<256, 256, 2, 4, EPI, BIAS>(p, st);
    return;
  }
  p.tiles_m = (int)((p.m + 255) / 256);
  p.tiles_n = (int)((p.n + 255) / 256);
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
  const int64_t cus = compute_units() >= 8 ? compute_units() / 8 * 8 : 8;
  const dim3 grid((unsigned)(tiles < cus ? tiles : cus));
  if constexpr (EPI != EPI_RAW) {
    if (p.staged && p.n <= (1 << 21)) {  // the pass-staged epilogue's byte offsets stay below 2^31
      hipLaunchKernelGGL((gemm_stream<EPI, BIAS, true>), grid, dim3(512), 0, st, p);
      return;
    }
  }
  hipLaunchKernelGGL((gemm_stream<EPI, BIAS, false>), grid, dim3(512), 0, st, p);
}

template <int EPI, bool BIAS>
void launch_fast(int tile, GemmArgs& p, hipStream_t st) {
  switch (tile) {
    case LR_TILE_256x256_PERSISTENT: launch_persistent<EPI, BIAS>(p, st); break;
    // 8 waves of 128x64; three A and two W 32 KB k-steps in LDS; 1 block per
    // CU. The large shapes take it: with four waves across N each wave of the
    // ping-pong loop refills only W rows that it alone reads in its group.
    case LR_TILE_256x256: launch_fast_cfg<256, 256, 2, 4, EPI, BIAS>(p, st); break;
    // 8 waves of 64x128 (same block shape, other wave grid; its W refill waits
    // for a barrier, 3-4% slower at the FFN-up shape).
    case LR_TILE_256x256_W4x2: launch_fast_cfg<256, 256, 4, 2, EPI, BIAS>(p, st); break;
    // 8 waves of 64x96: 192-column tiles fill the CUs where 256-column ones leave a
    // partial wave (N = 5120 at M = 2048: 216 tiles instead of 160).
    case LR_TILE_256x192: launch_fast_cfg<256, 192, 4, 2, EPI, BIAS>(p, st); break;
    // 4 waves of 128x64 / 64x128; two 48 KB k-steps.
    case LR_TILE_256x128: launch_fast_cfg<256, 128, 2, 2, EPI, BIAS>(p, st); break;
    case LR_TILE_128x256: launch_fast_cfg<128, 256, 2, 2, EPI, BIAS>(p, st); break;
    // 4 waves of 64x64; 80 KB of rings: 2 blocks per CU.
    case LR_TILE_128x128: launch_fast_cfg<128, 128, 2, 2, EPI, BIAS>(p, st); break;
    // 4 waves of 64x32 (24 KB k-steps), both operands GEMM_DEPTH_SMALL - 1
    // k-steps ahead: small-M GEMMs are bound by the DMA latency of their few
    // tiles, not by LDS or MFMA.
    // Weight-streaming tiles for a few hundred rows: 4 waves of 64x80 (or
    // 16x80). 256x80 makes one wave of tiles from N = 20480 at M <= 256, 64x80
    // one wave from N = 5120 at M <= 256. 256x80 takes 4 + 3 slots (158 KB; A
    // re-read from L2 by every CU dominates). 64x80 takes 4 + 4 (72 KB, both
    // rings 3 k-steps ahead). Graph-replayed at N = K = 5120, forced 64x80:
    // 13.7-13.8 us at M = 256 against 14.3 for 8 + 8, 11.2-11.3 against 11.8
    // at M = 64, 4-5% on every shape measured from M = 1 to 256. Where the
    // tiles spill past one wave, two 72 KB blocks share a CU: M = 256,
    // N = 5376, K = 7168 26.7 against 31.2 us. 2 + 2 runs 60% slower; 4 + 8,
    // 8 + 4 and 8 + 8 land between; 6 + 6 and 7 + 7 are 12-20% slower than
    // 8 + 8, and so were 6 + 10, 9 + 7 and 10 + 6 on an earlier build.
    case LR_TILE_256x80: launch_fast_cfg<256, 80, GEMM_SKINNY_WAVES, 1, EPI, BIAS, GEMM_SKINNY_NA, GEMM_SKINNY_NB>(p, st); break;
    case LR_TILE_64x80: launch_fast_cfg<64, 80, 4, 1, EPI, BIAS, GEMM_SKINNY64_NA, GEMM_SKINNY64_NB>(p, st); break;
    // 4 waves of 64x80 over 128 rows: one wave of tiles from N = 20480 at
    // M <= 256 that moves 36 KB per k-step against 44 KB for 256x80 (every CU
    // re-reads its A rows from L2): 29 against 34 us at M = 256. 4 + 4 slots
    // (144 KB).
    case LR_TILE_128x160: launch_fast_cfg<128, 160, 2, 2, EPI, BIAS, GEMM_SKINNY128_NA, GEMM_SKINNY128_NB>(p, st); break;
    // 8 waves of 96x64 (the 2x4 grid, so the early W refill): where 256x256
    // tiles leave the last wave a quarter empty (M = 12288, N = 5120: 960
    // tiles = 3.75 waves) its 1280 tiles make 5 full waves. Each tile carries
    // more fixed cost per op, so it pays only at long K: FFN-down (K = 20480)
    // 865 against 881 us, out-proj (K = 5120) 231 against 224 us.
    case LR_TILE_192x256: launch_fast_cfg<192, 256, 2, 4, EPI, BIAS>(p, st); break;
    default: launch_fast_cfg<64, 128, 1, 4, EPI, BIAS, GEMM_DEPTH_SMALL, GEMM_DEPTH_SMALL>(p, st); break;
  }
}

template <int EPI, bool BIAS>
void launch_generic(GemmArgs& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.n + 63) / 64), (unsigned)((p.m + 63) / 64));
  hipLaunchKernelGGL((gemm_generic<EPI, BIAS>), grid, dim3(256), 0, st, p);
}

// The split-K pass: the tile's raw-int32 kernel over tiles x splits workgroups
// into the workspace, then splitk_reduce with the caller's epilogue.
template <int EPI, bool BIAS>
void launch_split(int tile, GemmArgs p, int32_t* ws, hipStream_t st) {
  GemmArgs q = p;
  q.c = ws;
  q.bias = nullptr;
  q.nvec = 1;  // N % 4 == 0 and a 256-byte aligned workspace
  q.staged = 0;
  launch_fast<EPI_RAW, false>(tile, q, st);
  const int splits = p.splits;
  p.splits = 1;
  // The 8-wide vector path also loads bias as 16-byte rows.
  p.staged = p.staged && (!BIAS || aligned(p.bias, 16));
  const int64_t threads = p.staged ? p.m * (p.n / 8) : p.m * p.n;
  hipLaunchKernelGGL((splitk_reduce<EPI, BIAS>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     p, (const int32_t*)ws, splits);
}

template <int EPI>
void dispatch_bias(bool generic, int tile, bool bias, GemmArgs& p, hipStream_t st) {
  if (generic) {
    if (bias) launch_generic<EPI, true>(p, st);
    else launch_generic<EPI, false>(p, st);
  } else {
    if (bias) launch_fast<EPI, true>(tile, p, st);
    else launch_fast<EPI, false>(tile, p, st);
  }
}

int tile_rows(int tile) {
  switch (tile) {
    case LR_TILE_256x256: case LR_TILE_256x256_W4x2: case LR_TILE_256x128: case LR_TILE_256x192:
    case LR_TILE_256x256_PERSISTENT:
      return 256;
    case LR_TILE_256x80: return 256;
    case LR_TILE_192x256: return 192;
    case LR_TILE_128x256: case LR_TILE_128x128: case LR_TILE_128x160: return 128;
    default: return 64;
  }
}
int tile_cols(int tile) {
  switch (tile) {
    case LR_TILE_256x256: case LR_TILE_256x256_W4x2: case LR_TILE_128x256: case LR_TILE_192x256:
    case LR_TILE_256x256_PERSISTENT:
      return 256;
    case LR_TILE_256x192: return 192;
    case LR_TILE_256x80: case LR_TILE_64x80: return 80;
    case LR_TILE_128x160: return 160;
    default: return 128;
  }
}

// Shape heuristic from measured sweeps on MI355X (256 CUs, K = 5120 and
// 20480, M from 64 to 12288, N from 5120 to 20480). A launch takes as many
// waves of tiles as its tile count fills the resident blocks of the device's
// CUs (one 256x256, 192x256, 256x192 or 64x128 block per CU, two 128x128
// blocks; a partitioned GPU has fewer CUs per device); each wave
// costs a weight per tile (below), and the fewest weighted waves win, ties to
// the larger tile. Past that, 256x256 and 192x256 are compared by a per-tile
// time in K (long K favours 192x256 when it fills the waves better).
int auto_tile(int64_t m, int64_t n, int64_t k) {
  const int64_t cus = compute_units();
  auto tiles = [&](int t) { return ((m + tile_rows(t) - 1) / tile_rows(t)) * ((n + tile_cols(t) - 1) / tile_cols(t)); };
  // A few hundred rows (graph-replay timings at K = 5120): 64x80 when its
  // tiles fit one wave (M = 256, N = 5120: 14.6 us against 16.2 us for
  // 64x128; M = 128, N = 10240: 14.7 against 16.6; M = 96, N = 7168: 13.7
  // against 14.9), except a nearly full wave at M <= 64, where 64x128 is 3%
  // ahead (M = 64, N = 20480: 19.2 against 19.8 us). Where 64x80 tiles spill
  // past one wave but 64x128 tiles fit it, 64x128 (M = 256, N = 5376: 168
  // tiles, 19.5 us against 28.8 us for 128x160's 68 tiles at K = 7168, 35.3
  // against 51.5 us at K = 14336). Else 128x160 when its tiles fit one wave
  // (M = 256, N = 20480: 29 us against 34 us for 256x80 and 38 us for
  // 128x128).
  if (m <= 256) {
    if (tiles(LR_TILE_64x80) <= (m <= 64 ? cus * 3 / 4 : cus)) return LR_TILE_64x80;
    if (tiles(LR_TILE_64x128) <= cus) return LR_TILE_64x128;
    if (m > 128 && tiles(LR_TILE_128x160) <= cus) return LR_TILE_128x160;
  }
  // Relative cost of a wave of tiles (one per CU; two per CU for 128x128).
  // The 192-row and 192-column tiles hold the same outputs; 192x256 runs the
  // 2x4 wave grid, whose W refill goes out a phase earlier than the 4x2 grid
  // of 256x192, and is taken unless it needs more waves. Graph-replayed at
  // K = 5120 on M = 512-6144, N = 5120-20480 and K = 20480 on N = 5120, these
  // weights pick the fastest tile or one within 0.6% on all 24 shapes (M =
  // 2048, N = 5120: 47.0 us against 48.0 for 256x192; M = 4096, N = 5120:
  // 90.4 us against 97.4 for 128x128, whose wave is 0.74 of a 192-row one).
  auto waves = [&](int t, int64_t slots) { return (tiles(t) + slots - 1) / slots; };
  const int64_t w192w = waves(LR_TILE_256x192, cus), w192t = waves(LR_TILE_192x256, cus);
  const int64_t c256 = waves(LR_TILE_256x256, cus) * 66;
  const int64_t c192 = (w192t <= w192w ? w192t : w192w) * 60;
  const int64_t c128 = waves(LR_TILE_128x128, 2 * cus) * 44;
  const int64_t c64 = waves(LR_TILE_64x128, cus) * 22;
  if (c192 < c256 && c192 < c128 && c192 < c64) return w192t <= w192w ? LR_TILE_192x256 : LR_TILE_256x192;
  if (c256 <= c128 && c256 <= c64) {
    // 192x256 against 256x256 by per-tile time a + b*K (us, fitted at K = 5120
    // and 20480 on M = 12288, N = 5120): a longer K spreads 192x256's larger
    // fixed cost per op and leaves the wave count to decide.
    const double t256 = (double)waves(LR_TILE_256x256, cus) * (1.3 + 0.01068 * (double)k);
    const double t192 = (double)waves(LR_TILE_192x256, cus) * (3.9 + 0.008255 * (double)k);
    return t192 < 0.99 * t256 ? LR_TILE_192x256 : LR_TILE_256x256;
  }
  return c128 <= c64 ? LR_TILE_128x128 : LR_TILE_64x128;
}

// Split-K for a few hundred rows at long K, on 128x160 tiles: as many slices
// as keep the workgroups within one wave of the device's CUs, at most 4 (1 =
// no split).
// Graph-replayed at M = 256, N = 5120, K = 20480 (bf16 + bias): 35.6 us for
// 128x160 in 4 slices against 41.8 us unsplit on the shape's own tile. At
// K = 5120 every split measured slower than the unsplit small-M tiles (the
// partial slices' write and re-read, and the second launch, cost more than
// the shorter k-loops save).
int auto_splits(int64_t m, int64_t n, int64_t k) {
  if (m > 256 || k < 16384 || k % 128 != 0 || n % 4 != 0) return 1;
  const int64_t tiles = ((m + 127) / 128) * ((n + 159) / 160);
  int64_t s = compute_units() / tiles;
  if (s > 4) s = 4;
  return s > 1 ? (int)s : 1;
}

}  // namespace
}  // namespace lr

using namespace lr;

namespace lr {
namespace {

// True when the MFMA fast path can run (W stored [N,K] row-major with 16-byte
// aligned rows; buffer descriptors need per-block ranges below 2^31 bytes).
bool fast_path(const int8_t* a, const int8_t* b, int64_t b_stride_k, int64_t b_stride_n, int64_t k,
               int tile) {
  return b_stride_k == 1 && b_stride_n == k && k % 16 == 0 && k > 0 && aligned(a, 16) &&
         aligned(b, 16) && k <= (1LL << 22) && tile != LR_TILE_GENERIC;
}

struct Plan {
  int tile;
  int splits;
};

// The fast-path schedule: the tile (LR_TILE_AUTO: by shape and epilogue) and
// the split-K factor (splits 0: by shape when a workspace is allowed, else 1).
// Where the shape takes 256x256 tiles over at least two waves of the chip and
// the epilogue is bf16 or GELU, the persistent grid with streamed tiles runs
// 1-2% faster than one tile per workgroup (QKV 12288x15360x5120: 660 against
// 672 us, FFN-up 894 against 902-914 us, the Flash model's QKV and out-proj
// shapes at full M likewise; same box). Its pass-staged gated epilogue is
// slower (out-proj 286 against 265 us), so the gated and raw epilogues keep
// one tile per workgroup.
Plan plan(int64_t m, int64_t n, int64_t k, int tile, int splits, bool workspace, int epilogue) {
  Plan pl{tile == LR_TILE_AUTO ? auto_tile(m, n, k) : tile, splits > 0 ? splits : 1};
  if (splits == 0 && workspace && tile == LR_TILE_AUTO) {
    const int s = auto_splits(m, n, k);
    if (s > 1) pl = Plan{LR_TILE_128x160, s};
  }
  if (tile == LR_TILE_AUTO && pl.tile == LR_TILE_256x256 && pl.splits == 1 &&
      (epilogue == LR_EPI_BF16 || epilogue == LR_EPI_GELU_TANH) && k % 128 == 0 && k >= 256 &&
      ((m + 255) / 256) * ((n + 255) / 256) >= 2 * (int64_t)compute_units())
    pl.tile = LR_TILE_256x256_PERSISTENT;
  return pl;
}

int64_t split_workspace(int64_t m, int64_t n, int splits) { return splits > 1 ? splits * m * n * 4 : 0; }

int gemm_impl(const int8_t* a, const int8_t* b, int64_t b_stride_k, int64_t b_stride_n, int64_t m,
              int64_t n, int64_t k, const float* row_scale, const float* col_scale, const void* bias,
              void* c, int epilogue, const void* residual, const void* table, int64_t table_rows,
              int64_t table_width, const int64_t* indices, int64_t sequence, int gate_slot,
              void* workspace, int64_t workspace_bytes, int splits, int tile, void* stream) {
  LR_REQUIRE(m >= 0 && n >= 0 && k >= 0, "int8_gemm: negative shape");
  LR_REQUIRE(epilogue >= LR_EPI_BF16 && epilogue <= LR_EPI_RAW_INT32,
             "int8_gemm: unknown epilogue %d", epilogue);
  LR_REQUIRE(tile >= LR_TILE_AUTO && tile <= LR_TILE_256x256_PERSISTENT, "int8_gemm: unknown tile %d",
             tile);
  LR_REQUIRE(splits >= 0 && splits <= 64, "int8_gemm: splits %d outside 0..64", splits);
  LR_REQUIRE(workspace_bytes >= 0 && (workspace != nullptr || workspace_bytes == 0),
             "int8_gemm: bad workspace");
  if (m == 0 || n == 0) return LR_OK;
  LR_REQUIRE(a && b && c, "int8_gemm: null A/B/C");
  if (epilogue != LR_EPI_RAW_INT32) LR_REQUIRE(row_scale && col_scale, "int8_gemm: null scales");
  if (epilogue == LR_EPI_GATED_RESIDUAL) {
    LR_REQUIRE(residual && table && indices, "int8_gemm: gated residual needs residual/table/indices");
    LR_REQUIRE(sequence > 0 && table_rows > 0 && gate_slot >= 0,
               "int8_gemm: bad gated-residual sequence/table/slot");
    LR_REQUIRE((int64_t)(gate_slot + 1) * n <= table_width,
               "int8_gemm: table width %lld too small for gate slot %d", (long long)table_width,
               gate_slot);
  }
  GemmArgs p{};
  p.a = a; p.b = b; p.rs = row_scale; p.cs = col_scale; p.bias = (const uint16_t*)bias;
  p.c = c; p.resid = (const uint16_t*)residual; p.table = (const uint16_t*)table;
  p.indices = indices; p.m = m; p.n = n; p.k = k; p.b_sk = b_stride_k; p.b_sn = b_stride_n;
  p.table_rows = table_rows; p.table_width = table_width; p.sequence = sequence;
  p.gate_slot = gate_slot;
  p.group_m = GEMM_GROUP_M;
  p.splits = 1;
  p.nvec = n % 4 == 0 && aligned(c, epilogue == LR_EPI_RAW_INT32 ? 16 : 8) &&
           (epilogue == LR_EPI_RAW_INT32 || aligned(col_scale, 16)) &&
           (bias == nullptr || aligned(bias, 8)) &&
           (epilogue != LR_EPI_GATED_RESIDUAL ||
            (aligned(residual, 8) && aligned(table, 8) && table_width % 4 == 0));

  p.staged = p.nvec && n % 8 == 0 && aligned(c, 16) &&
             (epilogue != LR_EPI_GATED_RESIDUAL ||
              (aligned(residual, 16) && aligned(table, 16) && table_width % 8 == 0));

  const bool fast = fast_path(a, b, b_stride_k, b_stride_n, k, tile);
  int32_t* ws = nullptr;
  if (!fast) {
    LR_REQUIRE((m + 63) / 64 <= 65535, "int8_gemm: generic path supports M <= 4194240");
    LR_REQUIRE(splits <= 1, "int8_gemm: split-K needs the MFMA fast path");
  } else {
    const Plan pl = plan(m, n, k, tile, splits, workspace != nullptr, epilogue);
    tile = pl.tile;
    const int64_t tiles = ((m + tile_rows(tile) - 1) / tile_rows(tile)) *
                          ((n + tile_cols(tile) - 1) / tile_cols(tile));
    LR_REQUIRE(tiles * pl.splits <= 0x7fffffffLL, "int8_gemm: too many tiles");
    if (pl.splits > 1) {
      LR_REQUIRE(tile != LR_TILE_256x256_PERSISTENT, "int8_gemm: the persistent tile does not split K");
      LR_REQUIRE(k % 128 == 0 && pl.splits <= k / 128,
                 "int8_gemm: split-K needs K %% 128 == 0 and at most K / 128 splits");
      LR_REQUIRE(n % 4 == 0, "int8_gemm: split-K needs N %% 4 == 0");
      const int64_t need = split_workspace(m, n, pl.splits);
      LR_REQUIRE(workspace_bytes >= need, "int8_gemm: %d-way split-K needs a %lld-byte workspace, got %lld",
                 pl.splits, (long long)need, (long long)workspace_bytes);
      LR_REQUIRE(aligned(workspace, 256), "int8_gemm: workspace must be 256-byte aligned");
      ws = static_cast<int32_t*>(workspace);
      p.splits = pl.splits;
    }
  }
  hipStream_t st = as_stream(stream);
  const bool has_bias = bias != nullptr && epilogue != LR_EPI_RAW_INT32;
  if (ws != nullptr) {
    switch (epilogue) {
      case LR_EPI_BF16:
        if (has_bias) launch_split<EPI_BF16, true>(tile, p, ws, st);
        else launch_split<EPI_BF16, false>(tile, p, ws, st);
        break;
      case LR_EPI_GELU_TANH:
        if (has_bias) launch_split<EPI_GELU, true>(tile, p, ws, st);
        else launch_split<EPI_GELU, false>(tile, p, ws, st);
        break;
      case LR_EPI_GATED_RESIDUAL:
        if (has_bias) launch_split<EPI_GATED, true>(tile, p, ws, st);
        else launch_split<EPI_GATED, false>(tile, p, ws, st);
        break;
      default: launch_split<EPI_RAW, false>(tile, p, ws, st); break;
    }
    return check_launch("int8_gemm");
  }
  switch (epilogue) {
    case LR_EPI_BF16: dispatch_bias<EPI_BF16>(!fast, tile, has_bias, p, st); break;
    case LR_EPI_GELU_TANH: dispatch_bias<EPI_GELU>(!fast, tile, has_bias, p, st); break;
    case LR_EPI_GATED_RESIDUAL: dispatch_bias<EPI_GATED>(!fast, tile, has_bias, p, st); break;
    default: dispatch_bias<EPI_RAW>(!fast, tile, false, p, st); break;
  }
  return check_launch("int8_gemm");
}

}  // namespace
}  // namespace lr

extern "C" int lr_int8_gemm(const int8_t* a, const int8_t* b, int64_t b_stride_k,
                            int64_t b_stride_n, int64_t m, int64_t n, int64_t k,
                            const float* row_scale, const float* col_scale, const void* bias,
                            void* c, int epilogue, const void* residual, const void* table,
                            int64_t table_rows, int64_t table_width, const int64_t* indices,
                            int64_t sequence, int gate_slot, int tile, void* stream) {
  return gemm_impl(a, b, b_stride_k, b_stride_n, m, n, k, row_scale, col_scale, bias, c, epilogue,
                   residual, table, table_rows, table_width, indices, sequence, gate_slot, nullptr, 0,
                   1, tile, stream);
}

extern "C" int lr_int8_gemm_ws(const int8_t* a, const int8_t* b, int64_t b_stride_k,
                               int64_t b_stride_n, int64_t m, int64_t n, int64_t k,
                               const float* row_scale, const float* col_scale, const void* bias,
                               void* c, int epilogue, const void* residual, const void* table,
                               int64_t table_rows, int64_t table_width, const int64_t* indices,
                               int64_t sequence, int gate_slot, void* workspace,
                               int64_t workspace_bytes, int splits, int tile, void* stream) {
  return gemm_impl(a, b, b_stride_k, b_stride_n, m, n, k, row_scale, col_scale, bias, c, epilogue,
                   residual, table, table_rows, table_width, indices, sequence, gate_slot, workspace,
                   workspace_bytes, splits, tile, stream);
}

// ------------------------------------------------ allocation-free entry ----
// Scratch of lr_int8_gemm_noalloc: the split-K slices for callers that cannot
// allocate (code under graph capture, tight serving loops). Each GPU the
// library runs on holds its own copy until the process ends. Every call on a
// GPU shares that GPU's copy, so calls that overlap on one GPU race. Nothing
// in it has to start at zero: each slice element is written by its split
// before the reduce kernel reads it.
constexpr int64_t kScratchBytes = 32LL << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64];

// The device address of `scratch` on the stream's device, looked up once per
// device with that device current (in host code the array's name is a
// host-side stand-in, not a device address).
int scratch_address(hipStream_t st, void** out) {
  int dev = 0;
  hipError_t e = hipStreamGetDevice(st, &dev);
  if (e != hipSuccess) return hip_fail(e, "int8_gemm_noalloc: hipStreamGetDevice");
  if (dev < 0 || dev >= 64) return fail(LR_EUNSUPPORTED, "int8_gemm_noalloc: device %d not supported", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int current = 0;
    e = hipGetDevice(&current);
    if (e != hipSuccess) return hip_fail(e, "int8_gemm_noalloc: hipGetDevice");
    if (current != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return hip_fail(e, "int8_gemm_noalloc: hipSetDevice");
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t back = current != dev ? hipSetDevice(current) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "int8_gemm_noalloc: hipGetSymbolAddress(scratch)");
    if (back != hipSuccess) return hip_fail(back, "int8_gemm_noalloc: hipSetDevice");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return LR_OK;
}
}  // namespace

extern "C" int lr_int8_gemm_noalloc(const int8_t* a, const int8_t* b, int64_t b_stride_k,
                                    int64_t b_stride_n, int64_t m, int64_t n, int64_t k,
                                    const float* row_scale, const float* col_scale, const void* bias,
                                    void* c, int epilogue, const void* residual, const void* table,
                                    int64_t table_rows, int64_t table_width, const int64_t* indices,
                                    int64_t sequence, int gate_slot, int splits, int tile,
                                    void* stream) {
  LR_REQUIRE(splits >= 0 && splits <= 64, "int8_gemm: splits %d outside 0..64", splits);
  const int64_t need = m > 0 && n > 0 && k > 0 ? lr_int8_gemm_workspace_size(m, n, k, splits, tile) : 0;
  LR_REQUIRE(need <= kScratchBytes,
             "int8_gemm_noalloc: this split needs %lld bytes of scratch, above the %lld-byte maximum "
             "(lr_int8_gemm_ws takes a workspace of any size)",
             (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(as_stream(stream), &ws);
    if (rc != LR_OK) return rc;
  }
  return gemm_impl(a, b, b_stride_k, b_stride_n, m, n, k, row_scale, col_scale, bias, c, epilogue,
                   residual, table, table_rows, table_width, indices, sequence, gate_slot, ws,
                   need > 0 ? kScratchBytes : 0, splits, tile, stream);
}

extern "C" int64_t lr_int8_gemm_workspace_size(int64_t m, int64_t n, int64_t k, int splits, int tile) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 128 != 0 || n % 4 != 0 || splits < 0 || splits > 64 ||
      tile < LR_TILE_AUTO || tile > LR_TILE_256x256_PERSISTENT || tile == LR_TILE_GENERIC)
    return 0;
  return split_workspace(m, n, plan(m, n, k, tile, splits, true, LR_EPI_RAW_INT32).splits);
}
