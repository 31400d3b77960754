// elementwise.hip - gated residual, SwiGLU (+ INT8 quant) and GELU-tanh.
//
// Restates model/kernels.py:131-185 (_gated_residual_safe_kernel,
// _swiglu_kernel, _swiglu_quant_int8_kernel). All of them are HBM-bound:
// 16-byte loads and stores, one pass, no LDS except the per-row reduction of
// the fused quantizer.
#include "lr_device.h"
#include "lr_runtime.h"

namespace lr {
namespace {

constexpr int kThreads = 256;

// Splits the flat chunk index g (8 elements per chunk) into (row, chunk in
// row) for rows of `cpr` chunks, starting from the block's first row.
__device__ __forceinline__ void split_chunk(int64_t g, int64_t cpr, int64_t& row, int64_t& off) {
  const int64_t base = (int64_t)blockIdx.x * kThreads;
  row = base / cpr;  // uniform across the block
  off = g - row * cpr;
  while (off >= cpr) {
    off -= cpr;
    ++row;
  }
}

// ------------------------------------------------------ gated residual ----
// out = bf16(x + bf16(gate * u)), gate = table[tr, slot*H + c]; kernels.py:146-153.
struct GatedArgs {
  const uint16_t* x;
  const uint16_t* u;
  const uint16_t* table;
  const int64_t* indices;
  uint16_t* out;
  int64_t rows, sequence, hidden, table_rows, table_width;
  int slot;
};

__global__ __launch_bounds__(kThreads) void gated_residual_vec(GatedArgs p) {
  const int64_t cpr = p.hidden / 8;
  const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (g >= p.rows * cpr) return;
  int64_t row, c;
  split_chunk(g, cpr, row, c);
  const int64_t tr = clamp_index(p.indices[row % p.sequence], p.table_rows);
  const uint4 xv = load_nt(reinterpret_cast<const uint4*>(p.x) + g);
  const uint4 uv = load_nt(reinterpret_cast<const uint4*>(p.u) + g);
  const uint4 gv = *reinterpret_cast<const uint4*>(p.table + tr * p.table_width +
                                                   (int64_t)p.slot * p.hidden + 8 * c);
  float x[8], u[8], gt[8];
  unpack8(xv, x);
  unpack8(uv, u);
  unpack8(gv, gt);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = x[e] + round_bf(gt[e] * u[e]);
  store_nt(reinterpret_cast<uint4*>(p.out) + g, pack8(x));
}

__global__ __launch_bounds__(kThreads) void gated_residual_any(GatedArgs p) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= p.rows * p.hidden) return;
  const int64_t row = e / p.hidden, c = e - row * p.hidden;
  const int64_t tr = clamp_index(p.indices[row % p.sequence], p.table_rows);
  const float gate = bf_to_f(p.table[tr * p.table_width + (int64_t)p.slot * p.hidden + c]);
  const float v = bf_to_f(p.x[e]) + round_bf(gate * bf_to_f(p.u[e]));
  p.out[e] = (uint16_t)(pack_bf2(v, 0.0f) & 0xffffu);
}

// ------------------------------------------------------------- SwiGLU ----
// a = bf16(v * bf16(g * sigmoid(g))); kernels.py:156-185.
__device__ __forceinline__ float swiglu1(float v, float g) {
  return round_bf(v * round_bf(g * fast_sigmoid(g)));
}

__global__ __launch_bounds__(kThreads) void swiglu_vec(const uint16_t* __restrict__ p,
                                                       uint16_t* __restrict__ out, int64_t rows,
                                                       int64_t inner) {
  const int64_t cpr = inner / 8;
  const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (g >= rows * cpr) return;
  int64_t row, c;
  split_chunk(g, cpr, row, c);
  const uint16_t* prow = p + row * 2 * inner;
  float v[8], gt[8];
  unpack8(load_nt(reinterpret_cast<const uint4*>(prow + 8 * c)), v);
  unpack8(load_nt(reinterpret_cast<const uint4*>(prow + inner + 8 * c)), gt);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = swiglu1(v[e], gt[e]);
  store_nt(reinterpret_cast<uint4*>(out) + g, pack8(v));
}

__global__ __launch_bounds__(kThreads) void swiglu_any(const uint16_t* __restrict__ p,
                                                       uint16_t* __restrict__ out, int64_t rows,
                                                       int64_t inner) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= rows * inner) return;
  const int64_t row = e / inner, c = e - row * inner;
  const float a = swiglu1(bf_to_f(p[row * 2 * inner + c]), bf_to_f(p[row * 2 * inner + inner + c]));
  out[e] = (uint16_t)(pack_bf2(a, 0.0f) & 0xffffu);
}

template <int CPT>
__global__ __launch_bounds__(kThreads) void swiglu_quant_vec(const uint16_t* __restrict__ p,
                                                             uint2* __restrict__ q,
                                                             float* __restrict__ scales,
                                                             int64_t inner) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t cpr = inner / 8;
  const uint4* vrow = reinterpret_cast<const uint4*>(p + row * 2 * inner);
  const uint4* grow = reinterpret_cast<const uint4*>(p + row * 2 * inner + inner);
  float a[CPT][8];
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + i * kThreads;
    if (c < cpr) {
      float gt[8];
      unpack8(load_nt(vrow + c), a[i]);
      unpack8(load_nt(grow + c), gt);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a[i][e] = swiglu1(a[i][e], gt[e]);
        m = fmaxf(m, __builtin_fabsf(a[i][e]));
      }
    }
  }
  m = block256_max(m, red);
  const float s = quant_scale(m);
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + i * kThreads;
    if (c < cpr) q[row * cpr + c] = quant8(a[i], s, inv);
  }
  if (threadIdx.x == 0) scales[row] = s;
}

// Any inner size: the activation is recomputed in the second pass (same
// arithmetic, so the same values).
__global__ __launch_bounds__(kThreads) void swiglu_quant_any(const uint16_t* __restrict__ p,
                                                             int8_t* __restrict__ q,
                                                             float* __restrict__ scales,
                                                             int64_t inner) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* prow = p + row * 2 * inner;
  float m = 0.0f;
  for (int64_t c = threadIdx.x; c < inner; c += kThreads)
    m = fmaxf(m, __builtin_fabsf(swiglu1(bf_to_f(prow[c]), bf_to_f(prow[inner + c]))));
  m = block256_max(m, red);
  const float s = quant_scale(m);
  const float inv = 1.0f / s;
  for (int64_t c = threadIdx.x; c < inner; c += kThreads)
    q[row * inner + c] = (int8_t)quant_one(swiglu1(bf_to_f(prow[c]), bf_to_f(prow[inner + c])), s, inv);
  if (threadIdx.x == 0) scales[row] = s;
}

// ------------------------------------------------------------ GELU-tanh ----
__global__ __launch_bounds__(kThreads) void gelu_vec(const uint4* __restrict__ x,
                                                     uint4* __restrict__ out, int64_t chunks) {
  const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (g >= chunks) return;
  float f[8];
  unpack8(load_nt(x + g), f);
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = fast_gelu_tanh(f[e]);
  store_nt(out + g, pack8(f));
}

__global__ __launch_bounds__(kThreads) void gelu_any(const uint16_t* __restrict__ x,
                                                     uint16_t* __restrict__ out, int64_t count) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= count) return;
  out[e] = (uint16_t)(pack_bf2(fast_gelu_tanh(bf_to_f(x[e])), 0.0f) & 0xffffu);
}

// GELU-tanh + per-row INT8 quantizer in one pass over the FFN-up output:
// the GELU counterpart of swiglu_quant (the reference fuses its FFN
// activation into the re-quantizer the same way, model/kernels.py:169-185).
// Each value becomes bf16(gelu_tanh(x)) with fast_gelu_tanh, as the GEMM's
// GELU epilogue computes it, so gelu_quant(y) equals quantize_rows of that
// epilogue's output bit for bit. One block per row, the activated row in
// fp32 registers between the absmax and the quotient.
template <int CPT>
__global__ __launch_bounds__(kThreads) void gelu_quant_vec(const uint4* __restrict__ x,
                                                           uint2* __restrict__ q,
                                                           float* __restrict__ scales,
                                                           int64_t chunks) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint4* src = x + row * chunks;
  uint2* dst = q + row * chunks;
  uint4 v[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + i * kThreads;
    v[i] = c < chunks ? load_nt(src + c) : make_uint4(0, 0, 0, 0);
  }
  float a[CPT][8];
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    unpack8(v[i], a[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[i][e] = round_bf(fast_gelu_tanh(a[i][e]));  // gelu(0) = 0 past the row end
      m = fmaxf(m, __builtin_fabsf(a[i][e]));
    }
  }
  m = block256_max(m, red);
  const float s = quant_scale(m);
  const float inv = 1.0f / s;
  if (m < 0x1p80f) {  // the three-operation quotient (quantize.hip, norm.hip)
    const float lo = quant_lo(s, inv);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int64_t c = threadIdx.x + i * kThreads;
      if (c < chunks) dst[c] = quant8_split(a[i], inv, lo);
    }
  } else {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int64_t c = threadIdx.x + i * kThreads;
      if (c < chunks) dst[c] = quant8(a[i], s, inv);
    }
  }
  if (threadIdx.x == 0) scales[row] = s;
}

// Any width or alignment: the activation is recomputed in the second pass
// (same arithmetic, so the same values).
__global__ __launch_bounds__(kThreads) void gelu_quant_any(const uint16_t* __restrict__ x,
                                                           int8_t* __restrict__ q,
                                                           float* __restrict__ scales,
                                                           int64_t width) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* src = x + row * width;
  float m = 0.0f;
  for (int64_t c = threadIdx.x; c < width; c += kThreads)
    m = fmaxf(m, __builtin_fabsf(round_bf(fast_gelu_tanh(bf_to_f(src[c])))));
  m = block256_max(m, red);
  const float s = quant_scale(m);
  const float inv = 1.0f / s;
  for (int64_t c = threadIdx.x; c < width; c += kThreads)
    q[row * width + c] = (int8_t)quant_one(round_bf(fast_gelu_tanh(bf_to_f(src[c]))), s, inv);
  if (threadIdx.x == 0) scales[row] = s;
}

int blocks_for(int64_t work, unsigned* out) {
  const int64_t b = (work + kThreads - 1) / kThreads;
  if (b > 0x7fffffffLL) return fail(LR_EUNSUPPORTED, "elementwise: problem too large (not supported)");
  *out = (unsigned)b;
  return LR_OK;
}

}  // namespace
}  // namespace lr

using namespace lr;

extern "C" int lr_gated_residual(const void* x, const void* update, const void* table,
                                 const int64_t* indices, void* out, int64_t rows,
                                 int64_t sequence, int64_t hidden, int64_t table_rows,
                                 int64_t table_width, int gate_slot, void* stream) {
  LR_REQUIRE(rows >= 0 && hidden > 0 && sequence > 0, "gated_residual: bad shape");
  if (rows == 0) return LR_OK;
  LR_REQUIRE(x && update && table && indices && out, "gated_residual: null pointer");
  LR_REQUIRE(table_rows > 0 && gate_slot >= 0, "gated_residual: bad table/slot");
  LR_REQUIRE((int64_t)(gate_slot + 1) * hidden <= table_width,
             "gated_residual: table width %lld too small for slot %d", (long long)table_width,
             gate_slot);
  GatedArgs p{(const uint16_t*)x, (const uint16_t*)update, (const uint16_t*)table, indices,
              (uint16_t*)out, rows, sequence, hidden, table_rows, table_width, gate_slot};
  hipStream_t st = as_stream(stream);
  unsigned blocks;
  const bool vec = hidden % 8 == 0 && table_width % 8 == 0 && aligned(x, 16) &&
                   aligned(update, 16) && aligned(table, 16) && aligned(out, 16);
  int rc = blocks_for(vec ? rows * (hidden / 8) : rows * hidden, &blocks);
  if (rc) return rc;
  if (vec) hipLaunchKernelGGL(gated_residual_vec, dim3(blocks), dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL(gated_residual_any, dim3(blocks), dim3(kThreads), 0, st, p);
  return check_launch("gated_residual");
}

extern "C" int lr_swiglu(const void* p, void* out, int64_t rows, int64_t inner, void* stream) {
  LR_REQUIRE(rows >= 0 && inner >= 0, "swiglu: bad shape");
  if (rows == 0 || inner == 0) return LR_OK;
  LR_REQUIRE(p && out, "swiglu: null pointer");
  hipStream_t st = as_stream(stream);
  const bool vec = inner % 8 == 0 && aligned(p, 16) && aligned(out, 16);
  unsigned blocks;
  int rc = blocks_for(vec ? rows * (inner / 8) : rows * inner, &blocks);
  if (rc) return rc;
  if (vec)
    hipLaunchKernelGGL(swiglu_vec, dim3(blocks), dim3(kThreads), 0, st, (const uint16_t*)p,
                       (uint16_t*)out, rows, inner);
  else
    hipLaunchKernelGGL(swiglu_any, dim3(blocks), dim3(kThreads), 0, st, (const uint16_t*)p,
                       (uint16_t*)out, rows, inner);
  return check_launch("swiglu");
}

extern "C" int lr_swiglu_quant(const void* p, int8_t* q, float* scales, int64_t rows,
                               int64_t inner, void* stream) {
  LR_REQUIRE(rows >= 0 && inner > 0, "swiglu_quant: bad shape");
  if (rows == 0) return LR_OK;
  LR_REQUIRE(p && q && scales, "swiglu_quant: null pointer");
  LR_REQUIRE(rows <= 0x7fffffffLL, "swiglu_quant: too many rows");
  hipStream_t st = as_stream(stream);
  const int64_t cpr = inner / 8;
  const bool vec = inner % 8 == 0 && aligned(p, 16) && aligned(q, 8) && cpr <= 16 * kThreads;
  const dim3 grid((unsigned)rows), block(kThreads);
  if (vec) {
    const int64_t need = (cpr + kThreads - 1) / kThreads;
    if (need <= 1) hipLaunchKernelGGL(swiglu_quant_vec<1>, grid, block, 0, st, (const uint16_t*)p, (uint2*)q, scales, inner);
    else if (need <= 2) hipLaunchKernelGGL(swiglu_quant_vec<2>, grid, block, 0, st, (const uint16_t*)p, (uint2*)q, scales, inner);
    else if (need <= 4) hipLaunchKernelGGL(swiglu_quant_vec<4>, grid, block, 0, st, (const uint16_t*)p, (uint2*)q, scales, inner);
    else if (need <= 8) hipLaunchKernelGGL(swiglu_quant_vec<8>, grid, block, 0, st, (const uint16_t*)p, (uint2*)q, scales, inner);
    else hipLaunchKernelGGL(swiglu_quant_vec<16>, grid, block, 0, st, (const uint16_t*)p, (uint2*)q, scales, inner);
  } else {
    hipLaunchKernelGGL(swiglu_quant_any, grid, block, 0, st, (const uint16_t*)p, q, scales, inner);
  }
  return check_launch("swiglu_quant");
}

extern "C" int lr_gelu_tanh(const void* x, void* out, int64_t count, void* stream) {
  LR_REQUIRE(count >= 0, "gelu_tanh: bad count");
  if (count == 0) return LR_OK;
  LR_REQUIRE(x && out, "gelu_tanh: null pointer");
  hipStream_t st = as_stream(stream);
  const bool vec = count % 8 == 0 && aligned(x, 16) && aligned(out, 16);
  unsigned blocks;
  int rc = blocks_for(vec ? count / 8 : count, &blocks);
  if (rc) return rc;
  if (vec)
    hipLaunchKernelGGL(gelu_vec, dim3(blocks), dim3(kThreads), 0, st, (const uint4*)x,
                       (uint4*)out, count / 8);
  else
    hipLaunchKernelGGL(gelu_any, dim3(blocks), dim3(kThreads), 0, st, (const uint16_t*)x,
                       (uint16_t*)out, count);
  return check_launch("gelu_tanh");
}

extern "C" int lr_gelu_quant(const void* x, int8_t* q, float* scales, int64_t rows, int64_t width,
                             void* stream) {
  LR_REQUIRE(rows >= 0 && width > 0, "gelu_quant: bad shape");
  if (rows == 0) return LR_OK;
  LR_REQUIRE(x && q && scales, "gelu_quant: null pointer");
  LR_REQUIRE(rows <= 0x7fffffffLL, "gelu_quant: too many rows");
  hipStream_t st = as_stream(stream);
  const int64_t chunks = width / 8;
  const bool vec = width % 8 == 0 && aligned(x, 16) && aligned(q, 8) && chunks <= 16 * kThreads;
  const dim3 grid((unsigned)rows), block(kThreads);
  if (vec) {
    const int64_t need = (chunks + kThreads - 1) / kThreads;
    const uint4* src = static_cast<const uint4*>(x);
    uint2* dst = reinterpret_cast<uint2*>(q);
    if (need <= 1) hipLaunchKernelGGL(gelu_quant_vec<1>, grid, block, 0, st, src, dst, scales, chunks);
    else if (need <= 2) hipLaunchKernelGGL(gelu_quant_vec<2>, grid, block, 0, st, src, dst, scales, chunks);
    else if (need <= 4) hipLaunchKernelGGL(gelu_quant_vec<4>, grid, block, 0, st, src, dst, scales, chunks);
    else if (need <= 8) hipLaunchKernelGGL(gelu_quant_vec<8>, grid, block, 0, st, src, dst, scales, chunks);
    else if (need <= 10) hipLaunchKernelGGL(gelu_quant_vec<10>, grid, block, 0, st, src, dst, scales, chunks);
    else hipLaunchKernelGGL(gelu_quant_vec<16>, grid, block, 0, st, src, dst, scales, chunks);
  } else {
    hipLaunchKernelGGL(gelu_quant_any, grid, block, 0, st, static_cast<const uint16_t*>(x), q, scales,
                       width);
  }
  return check_launch("gelu_quant");
}
