// lr_device.h - device helpers shared by the gfx950 kernels of the W8A8 path.
//
// Every file that includes this is compiled with -ffp-contract=off and IEEE
// division/sqrt, so each `a * b + c` below is two roundings, exactly as in the
// reference's Triton kernels (compiled with enable_fp_fusion=False,
// model/int8_gemm.py:139,156; model/kernels.py:45,270) and its torch path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Streaming (non-temporal) 16-byte global load/store for data touched once.
__device__ __forceinline__ uint4 load_nt(const uint4* p) {
  v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt(uint4* p, uint4 v) {
  v4u w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<v4u*>(p));
}

// ---------------------------------------------------------------- bf16 ----
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf_to_f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Two floats -> packed bf16x2, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  v2f v = {lo, hi};
  v2bf b = __builtin_convertvector(v, v2bf);
  return __builtin_bit_cast(uint32_t, b);
}

// float -> nearest bf16 -> float.
__device__ __forceinline__ float round_bf(float x) { return bf_lo(pack_bf2(x, 0.0f)); }

// Unpack 8 bf16 held in a uint4 into floats.
__device__ __forceinline__ void unpack8(const uint4& v, float f[8]) {
  f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
  f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
  f[4] = bf_lo(v.z); f[5] = bf_hi(v.z);
  f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}

__device__ __forceinline__ uint4 pack8(const float f[8]) {
  uint4 v;
  v.x = pack_bf2(f[0], f[1]);
  v.y = pack_bf2(f[2], f[3]);
  v.z = pack_bf2(f[4], f[5]);
  v.w = pack_bf2(f[6], f[7]);
  return v;
}

// ------------------------------------------------------ INT8 quantizer ----
// Per-row scale of model/int8.py:66 (and kernels.py:13): max(absmax, 1e-8)/127
// in fp32 with an IEEE division.
__device__ __forceinline__ float quant_scale(float absmax) { return fmaxf(absmax, 1e-8f) / 127.0f; }

// q = clamp(rint_half_even(x / s), -127, 127) with x / s the IEEE fp32
// quotient (model/int8.py:67). `inv` is the rounded reciprocal of s.
//
// With q = x/s exact and u = 2^-24: fl(1/s) = (1/s)(1+e1), y = fl(x*fl(1/s))
// = q(1+e1)(1+e2) and fl(x/s) = q(1+e3), |ei| <= u, so
// |y - fl(x/s)| <= 3u|q| <= 2.27e-5 because |x| <= absmax bounds |q| by
// 127(1+2^-23). Unless y lies within 2^-14 (6.1e-5) of a half-integer, y and
// fl(x/s) therefore round to the same integer. Inside that window (exact ties
// are common among bf16 inputs) the IEEE quotient itself is rounded.
__device__ __forceinline__ int quant_one(float x, float s, float inv) {
  float y = x * inv;
  float n = __builtin_rintf(y);
  if (__builtin_fabsf(y - n) >= 0.5f - 0x1p-14f) n = __builtin_rintf(x / s);
  n = fminf(fmaxf(n, -127.0f), 127.0f);
  return (int)n;
}

__device__ __forceinline__ uint32_t pack_i8x4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)d << 24);
}

// Quantize 8 values to 8 int8 packed in a uint2.
__device__ __forceinline__ uint2 quant8(const float f[8], float s, float inv) {
  uint2 r;
  r.x = pack_i8x4(quant_one(f[0], s, inv), quant_one(f[1], s, inv), quant_one(f[2], s, inv),
                  quant_one(f[3], s, inv));
  r.y = pack_i8x4(quant_one(f[4], s, inv), quant_one(f[5], s, inv), quant_one(f[6], s, inv),
                  quant_one(f[7], s, inv));
  return r;
}

// ------------------------------------------------------- activations ----
// sigmoid(g) = 1 / (1 + 2^(-g*log2(e))) with the hardware exp2 and
// reciprocal (about 1 ulp each). Tolerance-level parity, like the
// reference's tl.sigmoid (model/kernels.py:165,177).
__device__ __forceinline__ float fast_sigmoid(float g) {
  float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

// gelu_tanh(x) = 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3).
// Uses 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)):
//   gelu_tanh(x) = x / (1 + 2^(x (c0 + c1 x^2))),
//   c0 = -2 sqrt(2/pi) log2(e), c1 = 0.044715 c0.
__device__ __forceinline__ float fast_gelu_tanh(float x) {
  const float c0 = -2.3022082f;
  const float c1 = -0.10294324f;
  float x2 = x * x;
  float t = x * (c0 + c1 * x2);
  float e = __builtin_amdgcn_exp2f(t);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// ------------------------------------------------------- reductions ----
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Butterfly sum over the wave: lane i adds lane i^o for o = 32..1. Because
// float addition is commutative, every lane ends with the value the tree
// s[i] += s[i+o] (i < o) leaves in s[0].
__device__ __forceinline__ float wave_tree_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, kWave);
  return v;
}

// Block-wide max over 256 threads; every thread gets the result.
__device__ __forceinline__ float block256_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  return v;
}

// Canonical sum of 256 per-thread partials (thread t holds slot t):
// s[i] += s[i+h] for h = 128, 64, 32, ..., 1; result s[0] broadcast.
__device__ __forceinline__ float block256_tree_sum(float v, float* red) {
  red[threadIdx.x] = v;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  float a = red[lane] + red[lane + 128];
  float b = red[lane + 64] + red[lane + 192];
  return wave_tree_sum(a + b);
}

__device__ __forceinline__ int64_t clamp_index(int64_t i, int64_t n) {
  return i < 0 ? 0 : (i >= n ? n - 1 : i);
}

}  // namespace lr
