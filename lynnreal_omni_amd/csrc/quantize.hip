// quantize.hip - per-row INT8 activation quantizer and the stand-alone
// INT32 -> bf16 dequant epilogue.
//
// quantize_rows restates model/int8.py:66-67 (the torch path; the Triton
// kernel model/kernels.py:8-16 computes the same values). Rows up to 8192
// wide: one wave per row, four rows per 256-thread block; lane l holds 16-byte
// chunks l, l+64, ... in registers, the absmax is a wave butterfly, and the
// row is quantized from registers and written with 8-byte stores. Wider rows:
// one 256-thread block per row, same scheme with a block reduction. HBM
// traffic is the algorithmic 3 bytes/element plus 4 bytes/row.
#include "lr_device.h"
#include "lr_runtime.h"

namespace lr {
namespace {

constexpr int kThreads = 256;

template <int CPL>
__global__ __launch_bounds__(kThreads) void quantize_rows_wave(const uint4* __restrict__ x,
                                                               uint2* __restrict__ q,
                                                               float* __restrict__ scales,
                                                               int64_t rows, int chunks) {
  const int lane = threadIdx.x & 63;
  const int64_t row = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
  if (row >= rows) return;  // whole wave
  // Buffer accesses: past the row end loads give zero and stores are dropped.
  const auto src = row_rsrc(x + row * chunks, 16 * (int64_t)chunks);
  const auto dst = row_rsrc(q + row * chunks, 8 * (int64_t)chunks);
  uint4 v[CPL];
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) v[i] = buf_load16(src, 16u * lane, 1024u * i);
#pragma unroll
  for (int i = 0; i < CPL; ++i) m = absmax8(v[i], m);
  const float s = quant_scale(wave_max(m));
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    buf_store8(dst, 8u * lane, 512u * i, quant8_bf(v[i], s, inv));
    __builtin_amdgcn_sched_barrier(0);
  }
  if (lane == 0) scales[row] = s;
}

template <int CPT>
__global__ __launch_bounds__(kThreads) void quantize_rows_vec(const uint4* __restrict__ x,
                                                              uint2* __restrict__ q,
                                                              float* __restrict__ scales,
                                                              int chunks) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint4* src = x + row * chunks;
  uint2* dst = q + row * chunks;
  uint4 v[CPT];
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * kThreads;
    v[i] = c < chunks ? load_nt(src + c) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) m = absmax8(v[i], m);
  m = block256_max(m, red);
  const float s = quant_scale(m);
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * kThreads;
    if (c < chunks) dst[c] = quant8_bf(v[i], s, inv);
  }
  if (threadIdx.x == 0) scales[row] = s;
}

// Any width / alignment: two passes over global memory, element-wise.
__global__ __launch_bounds__(kThreads) void quantize_rows_any(const uint16_t* __restrict__ x,
                                                              int8_t* __restrict__ q,
                                                              float* __restrict__ scales,
                                                              int64_t width) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* src = x + row * width;
  float m = 0.0f;
  for (int64_t c = threadIdx.x; c < width; c += kThreads) m = fmaxf(m, __builtin_fabsf(bf_to_f(src[c])));
  m = block256_max(m, red);
  const float s = quant_scale(m);
  const float inv = 1.0f / s;
  for (int64_t c = threadIdx.x; c < width; c += kThreads)
    q[row * width + c] = (int8_t)quant_one(bf_to_f(src[c]), s, inv);
  if (threadIdx.x == 0) scales[row] = s;
}

// fp16 and fp32 rows (the reference's Triton quantizer loads any float type
// as fp32, model/kernels.py:12): the same scale, and the IEEE quotient x / s
// itself (the corrected-reciprocal form above is proven for bf16 values
// only). One block per row, two passes over the row (the second from L2).
template <typename T>
__device__ __forceinline__ float as_float(T v) { return (float)v; }

template <typename T>
__global__ __launch_bounds__(kThreads) void quantize_rows_typed(const T* __restrict__ x,
                                                                int8_t* __restrict__ q,
                                                                float* __restrict__ scales,
                                                                int64_t width) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* src = x + row * width;
  float m = 0.0f;
  for (int64_t c = threadIdx.x; c < width; c += kThreads) m = fmaxf(m, __builtin_fabsf(as_float(src[c])));
  m = block256_max(m, red);
  const float s = quant_scale(m);
  for (int64_t c = threadIdx.x; c < width; c += kThreads) {
    const float v = __builtin_rintf(as_float(src[c]) / s);
    q[row * width + c] = (int8_t)fminf(fmaxf(v, -127.0f), 127.0f);
  }
  if (threadIdx.x == 0) scales[row] = s;
}

template <int CPT>
void launch_quant_vec(const void* x, int8_t* q, float* s, int64_t rows, int chunks,
                      hipStream_t st) {
  hipLaunchKernelGGL(quantize_rows_vec<CPT>, dim3((unsigned)rows), dim3(kThreads), 0, st,
                     (const uint4*)x, (uint2*)q, s, chunks);
}

template <int CPL>
void launch_quant_wave(const void* x, int8_t* q, float* s, int64_t rows, int chunks,
                       hipStream_t st) {
  hipLaunchKernelGGL(quantize_rows_wave<CPL>, dim3((unsigned)((rows + 3) / 4)), dim3(kThreads), 0,
                     st, (const uint4*)x, (uint2*)q, s, rows, chunks);
}

// ------------------------------------------------------------ epilogue ----
// out = bf16(((float)acc * as[r]) * ws[c] + bias[c]); model/kernels.py:27-38.
template <bool HAS_BIAS>
__global__ __launch_bounds__(kThreads) void epilogue4(const int4* __restrict__ acc,
                                                      const float* __restrict__ as,
                                                      const float* __restrict__ ws,
                                                      const uint16_t* __restrict__ bias,
                                                      uint2* __restrict__ out, int64_t groups,
                                                      int64_t n4) {
  const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (g >= groups) return;
  const int64_t r = g / n4;
  const int64_t c = (g - r * n4) * 4;
  const int4 a = acc[g];
  const float rs = as[r];
  const float4 cs = *reinterpret_cast<const float4*>(ws + c);
  float v0 = ((float)a.x * rs) * cs.x, v1 = ((float)a.y * rs) * cs.y;
  float v2 = ((float)a.z * rs) * cs.z, v3 = ((float)a.w * rs) * cs.w;
  if (HAS_BIAS) {
    const uint2 b = *reinterpret_cast<const uint2*>(bias + c);
    v0 = v0 + bf_lo(b.x); v1 = v1 + bf_hi(b.x);
    v2 = v2 + bf_lo(b.y); v3 = v3 + bf_hi(b.y);
  }
  out[g] = make_uint2(pack_bf2(v0, v1), pack_bf2(v2, v3));
}

__global__ __launch_bounds__(kThreads) void epilogue1(const int32_t* __restrict__ acc,
                                                      const float* __restrict__ as,
                                                      const float* __restrict__ ws,
                                                      const uint16_t* __restrict__ bias,
                                                      uint16_t* __restrict__ out, int64_t total,
                                                      int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= total) return;
  const int64_t r = e / n, c = e - r * n;
  float v = ((float)acc[e] * as[r]) * ws[c];
  if (bias) v = v + bf_to_f(bias[c]);
  out[e] = (uint16_t)(pack_bf2(v, 0.0f) & 0xffffu);
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_quantize_rows(const void* x, int64_t rows, int64_t width, int8_t* q,
                                float* scales, void* stream) {
  LR_REQUIRE(rows >= 0 && width >= 0, "quantize_rows: negative shape (%lld, %lld)",
             (long long)rows, (long long)width);
  if (rows == 0) return LR_OK;
  LR_REQUIRE(x && q && scales, "quantize_rows: null pointer");
  LR_REQUIRE(rows <= 0x7fffffffLL, "quantize_rows: too many rows (%lld)", (long long)rows);
  hipStream_t st = as_stream(stream);
  const int64_t chunks = width / 8;
  const bool vec = width % 8 == 0 && aligned(x, 16) && aligned(q, 8) && chunks <= 16 * kThreads &&
                   width > 0;
  if (vec && chunks <= 16 * 64) {
    const int need = (int)((chunks + 63) / 64);
    const int c = (int)chunks;
    if (need <= 1) launch_quant_wave<1>(x, q, scales, rows, c, st);
    else if (need <= 2) launch_quant_wave<2>(x, q, scales, rows, c, st);
    else if (need <= 3) launch_quant_wave<3>(x, q, scales, rows, c, st);
    else if (need <= 4) launch_quant_wave<4>(x, q, scales, rows, c, st);
    else if (need <= 6) launch_quant_wave<6>(x, q, scales, rows, c, st);
    else if (need <= 8) launch_quant_wave<8>(x, q, scales, rows, c, st);
    else if (need <= 10) launch_quant_wave<10>(x, q, scales, rows, c, st);
    else if (need <= 12) launch_quant_wave<12>(x, q, scales, rows, c, st);
    else launch_quant_wave<16>(x, q, scales, rows, c, st);
  } else if (vec) {
    const int need = (int)((chunks + kThreads - 1) / kThreads);
    const int c = (int)chunks;
    if (need <= 1) launch_quant_vec<1>(x, q, scales, rows, c, st);
    else if (need <= 2) launch_quant_vec<2>(x, q, scales, rows, c, st);
    else if (need <= 3) launch_quant_vec<3>(x, q, scales, rows, c, st);
    else if (need <= 4) launch_quant_vec<4>(x, q, scales, rows, c, st);
    else if (need <= 6) launch_quant_vec<6>(x, q, scales, rows, c, st);
    else if (need <= 8) launch_quant_vec<8>(x, q, scales, rows, c, st);
    else if (need <= 10) launch_quant_vec<10>(x, q, scales, rows, c, st);
    else if (need <= 12) launch_quant_vec<12>(x, q, scales, rows, c, st);
    else launch_quant_vec<16>(x, q, scales, rows, c, st);
  } else {
    hipLaunchKernelGGL(quantize_rows_any, dim3((unsigned)rows), dim3(kThreads), 0, st,
                       (const uint16_t*)x, q, scales, width);
  }
  return check_launch("quantize_rows");
}

extern "C" int lr_quantize_rows_typed(const void* x, int dtype, int64_t rows, int64_t width,
                                      int8_t* q, float* scales, void* stream) {
  LR_REQUIRE(dtype == LR_DTYPE_BF16 || dtype == LR_DTYPE_F16 || dtype == LR_DTYPE_F32,
             "quantize_rows: unknown dtype %d", dtype);
  if (dtype == LR_DTYPE_BF16) return lr_quantize_rows(x, rows, width, q, scales, stream);
  LR_REQUIRE(rows >= 0 && width >= 0, "quantize_rows: negative shape (%lld, %lld)",
             (long long)rows, (long long)width);
  if (rows == 0) return LR_OK;
  LR_REQUIRE(x && q && scales, "quantize_rows: null pointer");
  LR_REQUIRE(rows <= 0x7fffffffLL, "quantize_rows: too many rows (%lld)", (long long)rows);
  hipStream_t st = as_stream(stream);
  if (dtype == LR_DTYPE_F16)
    hipLaunchKernelGGL(quantize_rows_typed<_Float16>, dim3((unsigned)rows), dim3(kThreads), 0, st,
                       (const _Float16*)x, q, scales, width);
  else
    hipLaunchKernelGGL(quantize_rows_typed<float>, dim3((unsigned)rows), dim3(kThreads), 0, st,
                       (const float*)x, q, scales, width);
  return check_launch("quantize_rows");
}

extern "C" int lr_int8_epilogue(const int32_t* acc, const float* a_scale, const float* w_scale,
                                const void* bias, void* out, int64_t m, int64_t n,
                                void* stream) {
  LR_REQUIRE(m >= 0 && n >= 0, "int8_epilogue: negative shape");
  if (m == 0 || n == 0) return LR_OK;
  LR_REQUIRE(acc && a_scale && w_scale && out, "int8_epilogue: null pointer");
  hipStream_t st = as_stream(stream);
  const bool vec = n % 4 == 0 && aligned(acc, 16) && aligned(w_scale, 16) && aligned(out, 8) &&
                   (bias == nullptr || aligned(bias, 8));
  if (vec) {
    const int64_t groups = m * (n / 4);
    const int64_t blocks = (groups + kThreads - 1) / kThreads;
    LR_REQUIRE(blocks <= 0x7fffffffLL, "int8_epilogue: too large");
    if (bias)
      hipLaunchKernelGGL(epilogue4<true>, dim3((unsigned)blocks), dim3(kThreads), 0, st,
                         (const int4*)acc, a_scale, w_scale, (const uint16_t*)bias, (uint2*)out,
                         groups, n / 4);
    else
      hipLaunchKernelGGL(epilogue4<false>, dim3((unsigned)blocks), dim3(kThreads), 0, st,
                         (const int4*)acc, a_scale, w_scale, (const uint16_t*)bias, (uint2*)out,
                         groups, n / 4);
  } else {
    const int64_t total = m * n;
    const int64_t blocks = (total + kThreads - 1) / kThreads;
    LR_REQUIRE(blocks <= 0x7fffffffLL, "int8_epilogue: too large");
    hipLaunchKernelGGL(epilogue1, dim3((unsigned)blocks), dim3(kThreads), 0, st, acc, a_scale,
                       w_scale, (const uint16_t*)bias, (uint16_t*)out, total, n);
  }
  return check_launch("int8_epilogue");
}
