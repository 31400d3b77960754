// adaln.hip - the adaLN modulation table: a skinny bf16 GEMM over the
// time embeddings.
//
// Restates model/fusion.py:68-69 (fused_block) and elementwise_fusion.py:8-10:
//   table = adaln_proj.linear(F.silu(temb).to(bf16)).view(-1, 6 * hidden)
// i.e. out[m, n] = bf16(sum_k a[m, k] * W[n, k] + bias[n]) with
// a = bf16(silu(temb)) (silu = x / (1 + exp(-x)) in fp32, as torch computes
// it) and fp32 accumulation. M is the number of distinct time embeddings (a
// handful), K the embedding width, N = 6 * hidden: the launch streams W once
// and is HBM-bound on it (2 * N * K bytes).
//
// Layout: a block of 8 waves holds a for all M rows in LDS as bf16. Each
// wave takes whole output columns n (a W row, K contiguous bf16): lane l
// reads 16-byte chunks c = l, l + 64, ... of two columns at a time (one LDS
// read of a serves both; each column in two halves, the next half's loads in
// flight while the current one is summed) and accumulates, per row m and
// column, in
// chunk order and element order with fma (a bf16 x bf16 product is exact in
// fp32, so each step rounds once); the 64 lane partials are then combined by
// the butterfly tree s[i] += s[i + h], h = 32 .. 1, and bias is added.
#include "lr_device.h"
#include "lr_runtime.h"

namespace lr {
namespace {

constexpr int kAdalnThreads = 512;
constexpr int kAdalnMaxRows = 8;

struct AdalnArgs {
  const void* temb;
  const uint16_t* w;
  const uint16_t* bias;
  uint16_t* out;
  int64_t k, n;
  int temb_bf16, silu;
};

__device__ __forceinline__ float silu1(float x) { return x / (1.0f + expf(-x)); }

// Chunks [first, first + H) of column n, lane's share. Chunks past K, and
// every chunk of a column past the last (a zero-size descriptor), read as
// zero without touching memory, so the loads are issued unconditionally and
// the compiler can count them (a conditional load would make it wait for all).
template <int H>
__device__ __forceinline__ void load_part(const AdalnArgs& p, int64_t n, int first, int lane,
                                          uint4 (&w)[H]) {
  const bool live = n < p.n;
  const auto r = row_rsrc(p.w + (live ? n : 0) * p.k, live ? 2 * p.k : 0);
#pragma unroll
  for (int i = 0; i < H; ++i) w[i] = buf_load16(r, 16u * lane, 1024u * (first + i));
}

// F32: a is kept in LDS as fp32 (two float4 per chunk) instead of bf16, which
// saves the unpack of every read for a second LDS read; worth it from three
// rows on, where the unpacks dominate the VALU work.
template <int M, int CPL, bool F32>
__global__ __launch_bounds__(kAdalnThreads) void adaln_table(AdalnArgs p) {
  extern __shared__ uint4 a_lds[];  // [M][kc]: 8 bf16 per chunk, or 2 x 4 fp32 with F32
  const int kc = (int)(p.k / 8);
  for (int idx = threadIdx.x; idx < M * kc; idx += kAdalnThreads) {
    const int m = idx / kc, c = idx - m * kc;
    float x[8];
    if (p.temb_bf16) {
      unpack8(reinterpret_cast<const uint4*>(p.temb)[(int64_t)m * kc + c], x);
    } else {
      const float4* f = reinterpret_cast<const float4*>(p.temb) + 2 * ((int64_t)m * kc + c);
      const float4 lo = f[0], hi = f[1];
      x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
      x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
    }
    if (p.silu) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = silu1(x[e]);
    }
    if (F32) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = round_bf(x[e]);
      float4* f = reinterpret_cast<float4*>(a_lds) + 2 * idx;
      f[0] = make_float4(x[0], x[1], x[2], x[3]);
      f[1] = make_float4(x[4], x[5], x[6], x[7]);
    } else {
      a_lds[idx] = pack8(x);
    }
  }
  __syncthreads();

  // wave (and so every column index) is uniform: readfirstlane tells the
  // compiler, which then keeps the buffer descriptors in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t step = (int64_t)gridDim.x * (kAdalnThreads / 64);
  int64_t n = (int64_t)blockIdx.x * (kAdalnThreads / 64) + wave;
  if (n >= p.n) return;  // whole wave; no block barrier follows
  // Work unit = half the chunks of two columns (n and n + step: one LDS read
  // of a serves both; the second is zero past the last column). Two register
  // sets alternate, A for the first half and B for the second, so that one
  // set's loads are in flight while the other is summed, with no register
  // copies (a copy would have to wait for its load).
  constexpr int H = (CPL + 1) / 2;
  uint4 a0[H], a1[H], b0[H], b1[H];
  float acc0[M], acc1[M];
  auto sum = [&](const uint4 (&w0)[H], const uint4 (&w1)[H], int half) {
    // The LDS addresses repeat on every pass; an opaque lane index keeps the
    // compiler from hoisting all M * CPL reads of a out of the column loop
    // (which would need hundreds of registers).
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const int c = lane_v + 64 * (half * H + i);
      if (c < kc) {
        float f0[8], f1[8];
        unpack8(w0[i], f0);
        unpack8(w1[i], f1);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          float af[8];
          if (F32) {
            const float4* f = reinterpret_cast<const float4*>(a_lds) + 2 * (m * kc + c);
            const float4 lo = f[0], hi = f[1];
            af[0] = lo.x; af[1] = lo.y; af[2] = lo.z; af[3] = lo.w;
            af[4] = hi.x; af[5] = hi.y; af[6] = hi.z; af[7] = hi.w;
          } else {
            unpack8(a_lds[m * kc + c], af);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            acc0[m] = __builtin_fmaf(af[e], f0[e], acc0[m]);
            acc1[m] = __builtin_fmaf(af[e], f1[e], acc1[m]);
          }
        }
      }
      // One chunk at a time: without the fence the scheduler hoists every
      // LDS read of the unrolled loop and runs out of registers.
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Bias through a descriptor too (zero size without bias): an unconditional
  // load keeps the wait counts static.
  const auto rbias = row_rsrc(p.bias ? (const void*)p.bias : (const void*)p.w,
                              p.bias ? 2 * p.n : 0);
  load_part<H>(p, n, 0, lane, a0);
  load_part<H>(p, n + step, 0, lane, a1);
  while (true) {
    const uint16_t bias0_bits = __builtin_amdgcn_raw_buffer_load_b16(rbias, 0, (int)(2 * n), 0);
    const uint16_t bias1_bits =
        __builtin_amdgcn_raw_buffer_load_b16(rbias, 0, (int)(2 * (n + step)), 0);
    load_part<H>(p, n, H, lane, b0);
    load_part<H>(p, n + step, H, lane, b1);
#pragma unroll
    for (int m = 0; m < M; ++m) acc0[m] = acc1[m] = 0.0f;
    sum(a0, a1, 0);
    const int64_t next = n + 2 * step;
    load_part<H>(p, next, 0, lane, a0);         // zeros past the end
    load_part<H>(p, next + step, 0, lane, a1);
    sum(b0, b1, 1);
    const bool second = n + step < p.n;
    const float bias0 = bf_to_f(bias0_bits), bias1 = bf_to_f(bias1_bits);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float s0 = wave_tree_sum(acc0[m]);
      const float s1 = wave_tree_sum(acc1[m]);
      if (lane == m) p.out[(int64_t)m * p.n + n] = (uint16_t)(pack_bf2(s0 + bias0, 0.0f) & 0xffffu);
      if (lane == m && second)
        p.out[(int64_t)m * p.n + n + step] = (uint16_t)(pack_bf2(s1 + bias1, 0.0f) & 0xffffu);
    }
    if (next >= p.n) break;
    n = next;
  }
}

template <int M, int CPL, bool F32>
int launch_rows(const AdalnArgs& p, hipStream_t st) {
  const size_t lds = (size_t)M * (size_t)(p.k / 8) * (F32 ? 32 : 16);  // at most 160 KB
  if (lds > 65536) {  // above the default dynamic LDS limit (gfx950 has 160 KB per CU)
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&adaln_table<M, CPL, F32>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return hip_fail(e, "adaln_table: LDS size");
  }
  // A persistent grid of the blocks that fit at once (registers and LDS decide),
  // each looping over columns; never more blocks than column pairs of waves.
  const auto kernel = reinterpret_cast<const void*>(&adaln_table<M, CPL, F32>);
  int resident = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, kernel, kAdalnThreads, lds) !=
          hipSuccess || resident < 1) {
    (void)hipGetLastError();
    resident = 1;
  }
  constexpr int64_t kWaves = kAdalnThreads / 64;
  const int64_t want = (p.n + 2 * kWaves - 1) / (2 * kWaves);
  const int64_t cap = (int64_t)resident * compute_units();
  const int64_t blocks = want < cap ? want : cap;
  hipLaunchKernelGGL((adaln_table<M, CPL, F32>), dim3((unsigned)blocks), dim3(kAdalnThreads), lds, st, p);
  return check_launch("adaln_table");
}

template <int M, bool F32>
int launch_cpl(const AdalnArgs& p, hipStream_t st) {
  const int64_t need = (p.k / 8 + 63) / 64;
  switch (need) {
    case 1: return launch_rows<M, 1, F32>(p, st);
    case 2: return launch_rows<M, 2, F32>(p, st);
    case 3: return launch_rows<M, 3, F32>(p, st);
    case 4: return launch_rows<M, 4, F32>(p, st);
    case 5: return launch_rows<M, 5, F32>(p, st);
    case 6: return launch_rows<M, 6, F32>(p, st);
    case 7: return launch_rows<M, 7, F32>(p, st);
    case 8: return launch_rows<M, 8, F32>(p, st);
    case 9: return launch_rows<M, 9, F32>(p, st);
    case 10: return launch_rows<M, 10, F32>(p, st);
    case 11: return launch_rows<M, 11, F32>(p, st);
    case 12: return launch_rows<M, 12, F32>(p, st);
    case 13: return launch_rows<M, 13, F32>(p, st);
    case 14: return launch_rows<M, 14, F32>(p, st);
    case 15: return launch_rows<M, 15, F32>(p, st);
    default: return launch_rows<M, 16, F32>(p, st);
  }
}

// fp32 activations in LDS from three rows on, while they fit in 160 KB.
template <int M>
int launch_m(const AdalnArgs& p, hipStream_t st) {
  if (M >= 3 && (int64_t)M * p.k * 4 <= 160 * 1024) return launch_cpl<M, true>(p, st);
  return launch_cpl<M, false>(p, st);
}

int launch_group(const AdalnArgs& p, int rows, hipStream_t st) {
  switch (rows) {
    case 1: return launch_m<1>(p, st);
    case 2: return launch_m<2>(p, st);
    case 3: return launch_m<3>(p, st);
    case 4: return launch_m<4>(p, st);
    case 5: return launch_m<5>(p, st);
    case 6: return launch_m<6>(p, st);
    case 7: return launch_m<7>(p, st);
    default: return launch_m<8>(p, st);
  }
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_adaln_table(const void* temb, int temb_is_bf16, int apply_silu,
                              const void* weight, const void* bias, void* out, int64_t rows,
                              int64_t in_features, int64_t out_features, void* stream) {
  LR_REQUIRE(rows >= 0 && in_features >= 0 && out_features >= 0, "adaln_table: negative shape");
  if (rows == 0 || out_features == 0) return LR_OK;
  LR_REQUIRE(temb && weight && out, "adaln_table: null pointer");
  if (in_features == 0 || in_features % 8 != 0 || in_features > 8 * 64 * 16)
    return fail(LR_EUNSUPPORTED,
                "adaln_table: in_features %lld not supported (a multiple of 8, at most 8192)",
                (long long)in_features);
  if (!aligned(temb, 16) || !aligned(weight, 16))
    return fail(LR_EUNSUPPORTED, "adaln_table: temb and weight must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  AdalnArgs p{};
  p.w = (const uint16_t*)weight;
  p.bias = (const uint16_t*)bias;
  p.k = in_features;
  p.n = out_features;
  p.temb_bf16 = temb_is_bf16 ? 1 : 0;
  p.silu = apply_silu ? 1 : 0;
  const int64_t elem = temb_is_bf16 ? 2 : 4;
  for (int64_t r0 = 0; r0 < rows; r0 += kAdalnMaxRows) {
    const int group = (int)(rows - r0 < kAdalnMaxRows ? rows - r0 : kAdalnMaxRows);
    p.temb = (const char*)temb + r0 * in_features * elem;
    p.out = (uint16_t*)out + r0 * out_features;
    const int rc = launch_group(p, group, st);
    if (rc != LR_OK) return rc;
  }
  return LR_OK;
}
