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

// Raw buffer access to one row of `bytes` bytes: loads past the end return
// zero and stores past the end are dropped, so row tails need no branches.
typedef unsigned v2u __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// `voff` is the per-lane byte offset, `soff` a wave-uniform one (an SGPR or
// constant, so that unrolled chunk loops share one offset register).
// buf_load16 is for data read once (non-temporal); buf_load16_reused for data
// that many waves read again (gamma, table rows).
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                            uint32_t soff = 0) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2 /* nt */);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 buf_load16_reused(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                   uint32_t soff = 0) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
// Cache policies of the row stores (measured on MI355X at 12288 rows of
// 5120): 8-byte stores (int8 rows) go out non-temporal (nt), which took the
// fused norm + quant from 42 to 38 us and the 5120-wide quantizer from 31 to
// 29 us; 16-byte stores (bf16 rows) write through to system scope (sc0 sc1),
// 4% faster for the bf16 norm, where nt made it 10% slower. Either way no
// dirty output lines are left in L2 for the end-of-kernel write-back. Inside
// the projection chain, write-back int8 stores ran both norms 3-5 us faster
// but left the step time level (3.120-3.125 ms either way): the dirty lines'
// write-back lands in the GEMM that follows.
constexpr int kStore16Policy = 0x11;  // sc0 | sc1
constexpr int kStore8Policy = 0x2;    // nt
__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                            uint32_t soff, uint4 v) {
  const v4u w = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(w, r, voff, soff, kStore16Policy);
}
__device__ __forceinline__ void buf_store8(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                           uint32_t soff, uint2 v) {
  const v2u w = {v.x, v.y};
  __builtin_amdgcn_raw_buffer_store_b64(w, r, voff, soff, kStore8Policy);
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

// float -> nearest bf16 -> float. One v_cvt_pk_bf16_f32 with a zero low half:
// the packed word is then the rounded value's fp32 bit pattern.
__device__ __forceinline__ float round_bf(float x) { return __uint_as_float(pack_bf2(0.0f, x)); }

// Rounds two floats to bf16 with one instruction; returns the packed pair and
// writes the rounded values back.
__device__ __forceinline__ uint32_t round_bf2(float& a, float& b) {
  const uint32_t r = pack_bf2(a, b);
  a = bf_lo(r);
  b = bf_hi(r);
  return r;
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ void set_word(uint4& v, int i, uint32_t w) {
  if (i == 0) v.x = w; else if (i == 1) v.y = w; else if (i == 2) v.z = w; else v.w = w;
}

// Hide a value from the optimizer's common-subexpression elimination (no code).
__device__ __forceinline__ void opaque(uint4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

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
// quotient (model/int8.py:67), for a bf16 value x of a row whose absmax gave
// s = quant_scale(absmax), and inv = 1 / s (IEEE).
//
// q0 = x * inv can differ from fl(x / s) by an ulp or two, enough to move a
// result that lies on or next to a half-integer (exact ties are common among
// bf16 inputs). One Markstein correction, r = fma(-q0, s, x) (exact) and
// q1 = fma(r, inv, q0), removes that: rint(q1) equals the clamped
// rint(fl(x / s)) for every bf16 absmax and every bf16 x with |x| <= absmax,
// which tests/quant_division_check.c verifies exhaustively (about 10^9 pairs).
// The clamp is therefore never active. Adding 1.5 * 2^23 rounds q1 to an
// integer (half to even, as rint) and leaves it in the low bits of the sum,
// whose low byte is the int8 two's complement. A NaN ends as 0.
__device__ __forceinline__ float quant_quotient(float x, float s, float inv) {
  const float q0 = x * inv;
  const float r = __builtin_fmaf(-q0, s, x);
  return __builtin_fmaf(r, inv, q0);
}
__device__ __forceinline__ uint32_t quant_bits(float x, float s, float inv) {
  return __float_as_uint(quant_quotient(x, s, inv) + 0x1.8p23f);
}

__device__ __forceinline__ int quant_one(float x, float s, float inv) {
  return (int)(int8_t)(quant_bits(x, s, inv) & 0xffu);
}

// The same quotient in three operations for rows with absmax < 2^80: with
// hi = 1/s and lo = fma(-s, hi, 1) * hi, hi + lo is 1/s to about 2^-47
// relative, and rint(fma(x, hi, x * lo)) equals the clamped rint(fl(x / s))
// for every bf16 absmax below 2^80 and bf16 x with |x| <= absmax
// (tests/quant_division_check.c, exhaustive; from absmax 2^125 on lo is
// subnormal and a few pairs differ).
__device__ __forceinline__ float quant_lo(float s, float hi) { return __builtin_fmaf(-s, hi, 1.0f) * hi; }
__device__ __forceinline__ float quant_quotient_split(float x, float hi, float lo) {
  return __builtin_fmaf(x, hi, x * lo);
}

// Four quotients q0..q3 -> their rounded int8 values packed in one word: each
// v_add_f32 adds 1.5 * 2^23 and, through SDWA, writes the low byte of the sum
// straight into byte k of the result (the others kept), one instruction per
// value where the add and a v_perm gather took 1.75. The first write zeroes
// the rest of the word. Checked on gfx950 against the add + v_perm packing for
// 2^20 quotients in [-127.6, 127.6], every half-integer in [-128, 128] and its
// two neighbours, signed zeros, infinities and NaN: identical words.
__device__ __forceinline__ uint32_t magic_bytes4(float q0, float q1, float q2, float q3) {
  const float magic = 0x1.8p23f;
  uint32_t d;
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
      : "=v"(d) : "v"(q0), "v"(magic));
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "v"(q1), "v"(magic));
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "v"(q2), "v"(magic));
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(d) : "v"(q3), "v"(magic));
  return d;
}

// Quantize 8 values (bf16-exact floats) to 8 int8 packed in a uint2.
__device__ __forceinline__ uint2 quant8(const float f[8], float s, float inv) {
  float q[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) q[e] = quant_quotient(f[e], s, inv);
  return make_uint2(magic_bytes4(q[0], q[1], q[2], q[3]), magic_bytes4(q[4], q[5], q[6], q[7]));
}

__device__ __forceinline__ uint2 quant8_split(const float f[8], float hi, float lo) {
  float q[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) q[e] = quant_quotient_split(f[e], hi, lo);
  return make_uint2(magic_bytes4(q[0], q[1], q[2], q[3]), magic_bytes4(q[4], q[5], q[6], q[7]));
}

// Quantize the 8 bf16 of a uint4 to 8 int8 packed in a uint2.
__device__ __forceinline__ uint2 quant8_bf(const uint4& v, float s, float inv) {
  float f[8];
  unpack8(v, f);
  return quant8(f, s, inv);
}

// Max of |x| over the 8 bf16 of a uint4, folded into m.
__device__ __forceinline__ float absmax8(const uint4& v, float m) {
  m = fmaxf(fmaxf(m, __builtin_fabsf(bf_lo(v.x))), __builtin_fabsf(bf_hi(v.x)));
  m = fmaxf(fmaxf(m, __builtin_fabsf(bf_lo(v.y))), __builtin_fabsf(bf_hi(v.y)));
  m = fmaxf(fmaxf(m, __builtin_fabsf(bf_lo(v.z))), __builtin_fabsf(bf_hi(v.z)));
  m = fmaxf(fmaxf(m, __builtin_fabsf(bf_lo(v.w))), __builtin_fabsf(bf_hi(v.w)));
  return m;
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
  float t = x * __builtin_fmaf(c1, x2, c0);  // one rounding fewer than c0 + c1 * x2
  float e = __builtin_amdgcn_exp2f(t);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// Cross-lane partners without the LDS crossbar: lane l gets the value of
// lane l ^ o. 32 and 16 use the gfx950 permlane swaps, whose two results hold
// (v[l ^ o], v[l]) in some order, so only their sum or max is formed; 8 is a
// rotation by 8 within a 16-lane row; 4 is a half-row mirror (l -> 7 - l)
// followed by a quad reversal; 2 and 1 are quad permutations. Every source
// lane of these patterns exists, so bound_ctrl changes no value; it is set
// because it lets the compiler fold the move into the add, max or multiply
// that uses it (one v_add_f32_dpp instead of a v_mov_b32_dpp and a v_add_f32).
template <int O>
__device__ __forceinline__ float xor_partner(float v) {
  const int u = __float_as_int(v);
  if (O == 8) return __int_as_float(__builtin_amdgcn_mov_dpp(u, 0x128, 0xf, 0xf, true));
  if (O == 4) {
    const int m = __builtin_amdgcn_mov_dpp(u, 0x141, 0xf, 0xf, true);
    return __int_as_float(__builtin_amdgcn_mov_dpp(m, 0x1b, 0xf, 0xf, true));
  }
  if (O == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(u, 0x4e, 0xf, 0xf, true));
  return __int_as_float(__builtin_amdgcn_mov_dpp(u, 0xb1, 0xf, 0xf, true));
}

template <bool MAX>
__device__ __forceinline__ float wave_combine(float v) {
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
    v = MAX ? fmaxf(a, b) : a + b;
  }
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
    v = MAX ? fmaxf(a, b) : a + b;
  }
  v = MAX ? fmaxf(v, xor_partner<8>(v)) : v + xor_partner<8>(v);
  v = MAX ? fmaxf(v, xor_partner<4>(v)) : v + xor_partner<4>(v);
  v = MAX ? fmaxf(v, xor_partner<2>(v)) : v + xor_partner<2>(v);
  v = MAX ? fmaxf(v, xor_partner<1>(v)) : v + xor_partner<1>(v);
  return v;
}

// Max over the wave; every lane gets the result.
__device__ __forceinline__ float wave_max(float v) { return wave_combine<true>(v); }

// Butterfly sum over the wave: lane i adds lane i^o for o = 32..1. Because
// float addition is commutative, every lane ends with the value the tree
// s[i] += s[i+o] (i < o) leaves in s[0].
__device__ __forceinline__ float wave_tree_sum(float v) { return wave_combine<false>(v); }

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
