// qknorm.hip - fused per-head RMSNorm of Q and K with rotary embedding.
//
// Restates model/kernels.py:187-257 (_qk_norm_full_rope_paired_kernel,
// rotary_dim == head_dim) and :345-402 (_qk_norm_rope_kernel, rotary_dim <
// head_dim), launched from model/fusion.py:35-52 between the QKV projection
// and attention. Per (batch, token, head) row of Q, and of K with its own
// weight:
//   rstd = 1 / sqrt(sumsq(row) / head_dim + eps)
//   n[d] = bf16((row[d] * rstd) * weight[d])
//   d < rotary_dim, half = rotary_dim / 2, c/s = bf16(cos/sin[token, d]):
//     d <  half: out = bf16(bf16(n[d] * c) - bf16(n[d + half] * s))
//     d >= half: out = bf16(bf16(n[d] * c) + bf16(n[d - half] * s))
//   d >= rotary_dim: out = n[d]
//
// One row takes L = head_dim / 8 lanes (16 bytes of Q and of K each), so a
// wave holds 64 / L rows. The sum of squares follows the reference's ordered
// reduction (model/kernels.py:333-344, _sum128): 32-element chunks, each
// reduced by the tree s[i] += s[i + h], h = 16 .. 1, then the chunk sums by
// the same tree ((s0 + s2) + (s1 + s3) for four chunks). Lane j = 4c + a
// holds elements 32c + 8a + e, e < 8, so h = 16 and 8 pair lanes a ^ 2 and
// a ^ 1 element by element (DPP), h = 4, 2, 1 stay inside the lane, and the
// chunk tree pairs lanes j ^ 8 and j ^ 4. The rotary partner of chunk j is
// chunk j + D or j - D (D = rotary_dim / 16), fetched from that lane with
// DPP, so Q and K are each read once.
#include "lr_device.h"
#include "lr_runtime.h"

namespace lr {
namespace {

struct QkArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* qw;
  const uint16_t* kw;
  const float* cos;
  const float* sin;
  uint16_t* qo;
  uint16_t* ko;
  int64_t tokens, sequence, heads, q_ts, q_hs, k_ts, k_hs, head_dim, rotary_dim;
  float eps;
};

// n = bf16((x * rstd) * w) for the 8 elements of a chunk, packed.
__device__ __forceinline__ uint4 normalize8(const uint4& x, const uint4& w, float rstd) {
  float xf[8], wf[8];
  unpack8(x, xf);
  unpack8(w, wf);
#pragma unroll
  for (int e = 0; e < 8; ++e) xf[e] = (xf[e] * rstd) * wf[e];
  return pack8(xf);
}

// head_dim = 8L is a power of two, so s / head_dim is exactly s * (1 / head_dim)
// (both are the correctly rounded s * 2^-k); the multiply avoids the
// correctly rounded division's ten-instruction expansion.
template <int L>
__device__ __forceinline__ float rsqrt_row(float eps, float s) {
  static_assert((L & (L - 1)) == 0, "power-of-two head_dim");
  const float ms = s * (1.0f / (float)(8 * L)) + eps;
  return 1.0f / __builtin_sqrtf(ms);
}

// Sum of squares of the row whose 8-element slice this lane holds, in the
// order described at the top of the file. Squares of bf16 values are exact.
template <int L>
__device__ __forceinline__ float sumsq8(const uint4& x) {
  float v[8];
  unpack8(x, v);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = v[e] * v[e];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = v[e] + xor_partner<2>(v[e]);   // h = 16
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = v[e] + xor_partner<1>(v[e]);   // h = 8
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = v[e] + v[e + 4];                // h = 4
  v[0] = v[0] + v[2];
  v[1] = v[1] + v[3];                                                // h = 2
  float s = v[0] + v[1];                                             // h = 1
  if (L >= 16) s = s + xor_partner<8>(s);                            // chunk c + 2
  if (L >= 8) s = s + xor_partner<4>(s);                             // chunk c + 1
  return s;
}

// n = bf16((x * rstd) * w) for the 8 elements of a chunk, as rounded floats.
__device__ __forceinline__ void normalize8f(const uint4& x, const uint4& w, float rstd, float n[8]) {
  float wf[8];
  unpack8(x, n);
  unpack8(w, wf);
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = round_bf((n[e] * rstd) * wf[e]);
}

// The rotary partner's rounded floats (no pack/unpack): chunk j < D pairs
// with chunk j + D, chunk j in [D, 2D) with j - D. A power-of-two D is the
// lane XOR j ^ D (DPP); any other D < 16 is a row shift of D lanes, down for
// the first half and up for the second (DPP row_shl / row_shr, which stay in
// the 16-lane row: j + D < 2D <= L <= 16 and j - D >= 0).
template <int D>
__device__ __forceinline__ float row_shift_partner(float v, bool first_half) {
  static_assert(D > 0 && D < 16, "row shift distance");
  const int u = __float_as_int(v);
  const int down = __builtin_amdgcn_mov_dpp(u, 0x100 + D, 0xf, 0xf, false);  // lane i <- i + D
  const int up = __builtin_amdgcn_mov_dpp(u, 0x110 + D, 0xf, 0xf, false);    // lane i <- i - D
  return __int_as_float(first_half ? down : up);
}

template <int D>
__device__ __forceinline__ void partner8(const float n[8], float np[8], bool first_half) {
  constexpr bool kXor = (D & (D - 1)) == 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (kXor) np[e] = xor_partner<D>(n[e]);
    else np[e] = row_shift_partner<D>(n[e], first_half);
  }
}

// L lanes per row (head_dim = 8L); D = rotary_dim / 16 (0: no rotary).
// One wave per token: it loads the token's cos/sin once (rounded to bf16,
// lanes j < 2D) and walks the token's heads RPW = 64 / L at a time, the next
// group's Q/K slices in flight while the current group is normalized and
// rotated. Loads and stores go through buffer descriptors that end at the
// token's last head, so heads past the end read zero and are not stored
// without any branch (a conditional memory access would make the compiler
// wait for every outstanding load).
template <int L, int D>
__global__ __launch_bounds__(256) void qk_norm_rope(QkArgs p) {
  constexpr int RPW = 64 / L;  // rows (heads) per wave step
  const int lane = threadIdx.x & 63;
  const int j = lane % L, sub = lane / L;
  const int64_t token = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (token >= p.tokens) return;  // whole wave
  const int64_t b = token / p.sequence, t = token - b * p.sequence;
  const auto rq = row_rsrc(p.q + b * p.sequence * p.q_ts + t * p.q_ts, 2 * p.heads * p.q_hs);
  const auto rk = row_rsrc(p.k + b * p.sequence * p.k_ts + t * p.k_ts, 2 * p.heads * p.k_hs);
  const auto rqo = row_rsrc(p.qo + token * p.heads * p.head_dim, 2 * p.heads * p.head_dim);
  const auto rko = row_rsrc(p.ko + token * p.heads * p.head_dim, 2 * p.heads * p.head_dim);
  const uint4 qw = *reinterpret_cast<const uint4*>(p.qw + 8 * j);
  const uint4 kw = *reinterpret_cast<const uint4*>(p.kw + 8 * j);
  float c[8], sn[8];
  if (D > 0 && j < 2 * D) {
    const float4* cr = reinterpret_cast<const float4*>(p.cos + t * p.rotary_dim + 8 * j);
    const float4* sr = reinterpret_cast<const float4*>(p.sin + t * p.rotary_dim + 8 * j);
    const float4 c0 = cr[0], c1 = cr[1], s0 = sr[0], s1 = sr[1];
    c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w; c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
    sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
    // The first half's out = a - bf16(p * s) is a + bf16(p * -s) exactly
    // (negation is exact and round-to-nearest-even is symmetric), so the sign
    // goes into sin once per token and the loop always adds.
    const bool first = j < D;
#pragma unroll
    for (int e = 0; e < 8; ++e) c[e] = round_bf(c[e]), sn[e] = first ? -round_bf(sn[e]) : round_bf(sn[e]);
  }
  // Byte offsets inside the token (the descriptors end at head `heads`).
  const uint32_t q_step = (uint32_t)(2 * RPW * p.q_hs), k_step = (uint32_t)(2 * RPW * p.k_hs);
  const uint32_t o_step = (uint32_t)(2 * RPW * p.head_dim);
  uint32_t q_off = (uint32_t)(2 * (sub * p.q_hs + 8 * j));
  uint32_t k_off = (uint32_t)(2 * (sub * p.k_hs + 8 * j));
  uint32_t o_off = (uint32_t)(2 * (sub * p.head_dim + 8 * j));
  uint4 qx = buf_load16(rq, q_off), kx = buf_load16(rk, k_off);
  for (int64_t h0 = 0; h0 < p.heads; h0 += RPW) {
    q_off += q_step;
    k_off += k_step;
    // The next group (zeros past the last head).
    const uint4 qn_x = buf_load16(rq, q_off), kn_x = buf_load16(rk, k_off);
    // Every lane takes part in the cross-lane steps; heads past the end hold zeros.
    const float q_rstd = rsqrt_row<L>(p.eps, sumsq8<L>(qx));
    const float k_rstd = rsqrt_row<L>(p.eps, sumsq8<L>(kx));
    uint4 qn, kn;
    if (D == 0) {
      qn = normalize8(qx, qw, q_rstd);
      kn = normalize8(kx, kw, k_rstd);
    } else {
      // Rounded floats throughout: the partner comes over DPP as floats, so
      // nothing is packed and unpacked again before the rotation.
      float nq[8], nk[8], pq[8], pk[8];
      normalize8f(qx, qw, q_rstd, nq);
      normalize8f(kx, kw, k_rstd, nk);
      const bool left = j < D;  // first half of the rotary dims: the partner is chunk j + D
      partner8<D>(nq, pq, left);
      partner8<D>(nk, pk, left);
      if (j < 2 * D) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          nq[e] = round_bf(nq[e] * c[e]) + round_bf(pq[e] * sn[e]);
          nk[e] = round_bf(nk[e] * c[e]) + round_bf(pk[e] * sn[e]);
        }
      }
      qn = pack8(nq);
      kn = pack8(nk);
    }
    buf_store16(rqo, o_off, 0, qn);
    buf_store16(rko, o_off, 0, kn);
    o_off += o_step;
    qx = qn_x;
    kx = kn_x;
  }
}

template <int L, int D>
void launch(const QkArgs& p, hipStream_t st) {
  const int64_t blocks = (p.tokens + 3) / 4;
  hipLaunchKernelGGL((qk_norm_rope<L, D>), dim3((unsigned)blocks), dim3(256), 0, st, p);
}

template <int L>
int launch_rot(const QkArgs& p, hipStream_t st) {
  // rotary_dim <= head_dim = 8L keeps the pair distance D = rotary_dim / 16 at most L / 2.
  switch (p.rotary_dim / 16) {
    case 0: launch<L, 0>(p, st); break;
    case 1: launch<L, 1>(p, st); break;
    case 2: launch<L, 2>(p, st); break;
    case 3: if constexpr (L >= 8) launch<L, 3>(p, st); break;
    case 4: if constexpr (L >= 8) launch<L, 4>(p, st); break;
    case 5: if constexpr (L >= 16) launch<L, 5>(p, st); break;
    case 6: if constexpr (L >= 16) launch<L, 6>(p, st); break;
    case 7: if constexpr (L >= 16) launch<L, 7>(p, st); break;
    case 8: if constexpr (L >= 16) launch<L, 8>(p, st); break;
    default: return fail(LR_EUNSUPPORTED, "qk_norm_rope: rotary_dim %lld not supported",
                         (long long)p.rotary_dim);
  }
  return check_launch("qk_norm_rope");
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_qk_norm_rope(const void* q, const void* k, const void* q_weight,
                               const void* k_weight, const float* cos, const float* sin,
                               void* q_out, void* k_out, int64_t batch, int64_t sequence,
                               int64_t heads, int64_t q_token_stride, int64_t q_head_stride,
                               int64_t k_token_stride, int64_t k_head_stride, int64_t head_dim,
                               int64_t rotary_dim, float eps, void* stream) {
  LR_REQUIRE(batch >= 0 && sequence >= 0 && heads >= 0, "qk_norm_rope: negative shape");
  const int64_t rows = batch * sequence * heads;
  if (rows == 0) return LR_OK;
  LR_REQUIRE(q && k && q_weight && k_weight && q_out && k_out, "qk_norm_rope: null pointer");
  LR_REQUIRE(rotary_dim >= 0 && rotary_dim <= head_dim && rotary_dim % 2 == 0,
             "qk_norm_rope: rotary dimensions must be even and fit the attention head");
  LR_REQUIRE(rotary_dim == 0 || (cos && sin), "qk_norm_rope: null cos/sin");
  if (!(head_dim == 32 || head_dim == 64 || head_dim == 128))
    return fail(LR_EUNSUPPORTED, "qk_norm_rope: head_dim %lld not supported (32, 64, 128)",
                (long long)head_dim);
  if (rotary_dim % 16 != 0)
    return fail(LR_EUNSUPPORTED, "qk_norm_rope: rotary_dim %lld not supported (a multiple of 16)",
                (long long)rotary_dim);
  const bool aligned_ok = aligned(q, 16) && aligned(k, 16) && aligned(q_weight, 16) &&
                          aligned(k_weight, 16) && aligned(q_out, 16) && aligned(k_out, 16) &&
                          q_token_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                          k_token_stride % 8 == 0 && k_head_stride % 8 == 0 &&
                          (rotary_dim == 0 || (aligned(cos, 16) && aligned(sin, 16)));
  if (!aligned_ok)
    return fail(LR_EUNSUPPORTED, "qk_norm_rope: rows must be 16-byte aligned");
  LR_REQUIRE((batch * sequence + 3) / 4 < 0x7fffffffLL, "qk_norm_rope: too many tokens");
  // Per-token descriptors: a token's heads must span less than 2^31 bytes.
  LR_REQUIRE(heads * (q_head_stride > k_head_stride ? q_head_stride : k_head_stride) <
                 (1LL << 30) - 64 * head_dim,
             "qk_norm_rope: a token's heads span too many bytes");
  LR_REQUIRE(q_head_stride >= head_dim && k_head_stride >= head_dim,
             "qk_norm_rope: heads must not overlap (head stride < head_dim)");
  QkArgs p{};
  p.q = (const uint16_t*)q; p.k = (const uint16_t*)k;
  p.qw = (const uint16_t*)q_weight; p.kw = (const uint16_t*)k_weight;
  p.cos = cos; p.sin = sin; p.qo = (uint16_t*)q_out; p.ko = (uint16_t*)k_out;
  p.tokens = batch * sequence; p.sequence = sequence; p.heads = heads;
  p.q_ts = q_token_stride; p.q_hs = q_head_stride; p.k_ts = k_token_stride; p.k_hs = k_head_stride;
  p.head_dim = head_dim; p.rotary_dim = rotary_dim; p.eps = eps;
  hipStream_t st = as_stream(stream);
  switch (head_dim) {
    case 32: return launch_rot<4>(p, st);
    case 64: return launch_rot<8>(p, st);
    default: return launch_rot<16>(p, st);
  }
}
