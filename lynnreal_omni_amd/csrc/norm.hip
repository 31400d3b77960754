// norm.hip - fused RMSNorm + adaLN modulate (+ gated residual) (+ INT8 quant).
//
// Restates model/kernels.py:48-128 (_rms_adaln_kernel and
// _rms_adaln_quant_int8_kernel, incl. its WITH_RESIDUAL branch :101-105).
// One 256-thread block owns one row (token). The row stays in registers from
// the first read to the last write, so HBM sees each byte once:
//   rms_adaln            2 B in + 2 B out per element
//   rms_adaln_quant      2 B in + 1 B out per element (+4 B/row)
//   residual_rms_quant   4 B in + 3 B out per element (+4 B/row)
// The gamma vector and the table rows are shared by all rows and stay in L2.
//
// The sum of squares uses one fixed order (8-element chunks, chunk j into
// slot j % 256, then a pairwise tree over the 256 slots), so a CPU
// restatement reproduces it bit for bit. The reference's Triton kernel sums
// in its own tree order with an approximate rsqrt; against it the bf16
// outputs agree to tolerance.
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
      // Each square of a bf16 is exact in fp32, so this is one rounding per add.
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = acc + v[i][e] * v[i][e];
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

template <bool RESID, bool QUANT>
int launch_norm(const NormArgs& p, int64_t rows, bool vec, hipStream_t st) {
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
