/*
 * lr_oracle.c - CPU restatement of LynnReal-Omni's W8A8 DiT projection path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the GPU kernels are
 * compared against; it is never part of the product path. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Each function cites the reference lines (relative to the reference
 * checkout) whose arithmetic it restates. bf16 values are IEEE bfloat16 bit
 * patterns held in uint16_t; conversions round to nearest even like
 * torch's c10::BFloat16 (NaN -> 0x7fc0).
 *
 * Build with -ffp-contract=off and without -ffast-math: every a*b+c below is
 * two roundings, as in the reference (enable_fp_fusion=False for Triton,
 * no contraction in torch's eager CPU ops).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------- bf16 --- */
static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float rbf(float f) { return bf2f(f2bf(f)); }

void lro_f32_to_bf16(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = f2bf(x[i]);
}

/* ----------------------------------------------- per-row quantizer --- */
/* model/int8.py:66-67:
 *   scale = flat.float().abs().amax(-1, keepdim=True).clamp_min_(1e-8) / 127
 *   quantized = (flat.float() / scale).round().clamp(-127, 127).to(torch.int8)
 * torch.round is round-half-to-even, as is rintf in the default FE mode. */
static void quant_row_f32(const float* v, int64_t width, int8_t* q, float* scale) {
  float m = 0.0f;
  for (int64_t c = 0; c < width; ++c) {
    const float a = fabsf(v[c]);
    if (a > m) m = a;
  }
  if (m < 1e-8f) m = 1e-8f;
  const float s = m / 127.0f;
  for (int64_t c = 0; c < width; ++c) {
    float t = rintf(v[c] / s);
    if (t > 127.0f) t = 127.0f;
    if (t < -127.0f) t = -127.0f;
    q[c] = (int8_t)t;
  }
  *scale = s;
}

void lro_quantize_rows(const uint16_t* x, int64_t rows, int64_t width, int8_t* q, float* scales) {
#pragma omp parallel
  {
    float* v = (float*)malloc(sizeof(float) * (width > 0 ? width : 1));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      for (int64_t c = 0; c < width; ++c) v[c] = bf2f(x[r * width + c]);
      quant_row_f32(v, width, q + r * width, scales + r);
    }
    free(v);
  }
}

/* ------------------------------------------------------ INT8 GEMM --- */
/* torch._int_mm(flat, weight_int8) of model/int8.py:51 / int8_gemm.py:87:
 * exact int32 accumulation. B[k, n] = b[k*bsk + n*bsn]; Int8Linear's
 * weight_int8 is a [K, N] view of [N, K] storage (bsk = 1, bsn = K). */
void lro_int_mm(const int8_t* a, const int8_t* b, int64_t bsk, int64_t bsn, int64_t m,
                int64_t n, int64_t k, int32_t* c) {
  if (bsk == 1) {
    /* W rows contiguous in k: dot products of two contiguous int8 rows. */
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t i = 0; i < m; ++i)
      for (int64_t j = 0; j < n; ++j) {
        const int8_t* ar = a + i * k;
        const int8_t* br = b + j * bsn;
        int32_t s = 0;
        for (int64_t t = 0; t < k; ++t) s += (int32_t)ar[t] * (int32_t)br[t];
        c[i * n + j] = s;
      }
  } else {
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t i = 0; i < m; ++i)
      for (int64_t j = 0; j < n; ++j) {
        int32_t s = 0;
        for (int64_t t = 0; t < k; ++t) s += (int32_t)a[i * k + t] * (int32_t)b[t * bsk + j * bsn];
        c[i * n + j] = s;
      }
  }
}

/* model/int8.py:55-58 (== int8_gemm.py:89-92 == kernels.py:33-38):
 *   output = acc.float() * scale.reshape(-1, 1).float() * weight_scale
 *   output = output + bias.float();  output.to(torch.bfloat16) */
void lro_dequant(const int32_t* acc, const float* rs, const float* cs, const uint16_t* bias,
                 int64_t m, int64_t n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float v = ((float)acc[i * n + j] * rs[i]) * cs[j];
      if (bias) v = v + bf2f(bias[j]);
      out[i * n + j] = f2bf(v);
    }
}

/* ------------------------------------------------------ activations --- */
/* GELU, tanh approximation: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))),
 * evaluated in double and rounded once to bf16. The reference has no in-tree
 * kernel for it; its only GELU-tanh INT8 path is comfy-kitchen's
 * int8_linear(input_act="gelu_tanh"), exercised at
 * comfyui/custom_nodes/ComfyUI-LynnReal/tools/verify_sampling_safety.py:59. */
static inline double gelu_tanh_d(double x) {
  const double k0 = 0.7978845608028654; /* sqrt(2/pi) */
  return 0.5 * x * (1.0 + tanh(k0 * (x + 0.044715 * x * x * x)));
}

void lro_gelu_tanh(const uint16_t* x, int64_t count, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) out[i] = f2bf((float)gelu_tanh_d((double)bf2f(x[i])));
}

/* SwiGLU, model/kernels.py:163-166 and :175-177:
 *   a = bf16(v * bf16(g * sigmoid(g)))   (sigmoid in double, product fp32) */
static inline float swiglu1(float v, float g) {
  const float sg = (float)(1.0 / (1.0 + exp(-(double)g)));
  return rbf(v * rbf(g * sg));
}

void lro_swiglu(const uint16_t* p, int64_t rows, int64_t inner, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < inner; ++c)
      out[r * inner + c] = f2bf(swiglu1(bf2f(p[r * 2 * inner + c]), bf2f(p[r * 2 * inner + inner + c])));
}

void lro_swiglu_quant(const uint16_t* p, int64_t rows, int64_t inner, int8_t* q, float* scales) {
#pragma omp parallel
  {
    float* v = (float*)malloc(sizeof(float) * (inner > 0 ? inner : 1));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      for (int64_t c = 0; c < inner; ++c)
        v[c] = swiglu1(bf2f(p[r * 2 * inner + c]), bf2f(p[r * 2 * inner + inner + c]));
      quant_row_f32(v, inner, q + r * inner, scales + r);
    }
    free(v);
  }
}

/* ------------------------------------------------- gated residual --- */
static inline int64_t clampi(int64_t i, int64_t n) { return i < 0 ? 0 : (i >= n ? n - 1 : i); }

/* model/kernels.py:144-153: out = bf16(x + bf16(gate * u)),
 * gate = table[indices[row % sequence], slot * hidden + c]. */
void lro_gated_residual(const uint16_t* x, const uint16_t* u, const uint16_t* table,
                        const int64_t* indices, int64_t rows, int64_t sequence, int64_t hidden,
                        int64_t table_rows, int64_t table_width, int slot, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t tr = clampi(indices[r % sequence], table_rows);
    const uint16_t* g = table + tr * table_width + (int64_t)slot * hidden;
    for (int64_t c = 0; c < hidden; ++c) {
      const int64_t e = r * hidden + c;
      out[e] = f2bf(bf2f(x[e]) + rbf(bf2f(g[c]) * bf2f(u[e])));
    }
  }
}

/* ------------------------------------- RMSNorm + adaLN (+ quant) --- */
/* Sum of squares in the order defined for the fused norm kernels: chunk j
 * (elements 8j .. 8j+7) goes to slot j % 256, each slot accumulates its
 * chunks in increasing j in fp32 as s = fmaf(x, x, s) (the square of a bf16
 * is exact in fp32 unless |x| < 2^-67, so this is s + x*x rounded once), and
 * the 256 slots are combined by s[i] += s[i + h] for h = 128, 64, ..., 1. */
static float canonical_sumsq(const float* v, int64_t hidden) {
  float slot[256];
  for (int i = 0; i < 256; ++i) slot[i] = 0.0f;
  const int64_t chunks = (hidden + 7) / 8;
  for (int64_t j = 0; j < chunks; ++j) {
    float acc = slot[j % 256];
    for (int64_t e = 8 * j; e < 8 * j + 8 && e < hidden; ++e) acc = fmaf(v[e], v[e], acc);
    slot[j % 256] = acc;
  }
  for (int h = 128; h >= 1; h >>= 1)
    for (int i = 0; i < h; ++i) slot[i] = slot[i] + slot[i + h];
  return slot[0];
}

/* model/kernels.py:59-78 and :95-128 (incl. the residual branch :101-105):
 *   (residual) x' = bf16(x + bf16(table[tr, 2H + c] * u)), stored
 *   rr = 1 / sqrt(sumsq(x) / H + eps)
 *   n  = bf16((x * rr) * w)
 *   y  = bf16(bf16(n * bf16(1 + scale)) + shift)
 *   (quant) q, s = per-row quantizer of model/int8.py:66-67 applied to y
 * mode: 0 = bf16 out, 1 = quant, 2 = residual + quant. */
static void rms_adaln_impl(const uint16_t* x, const uint16_t* u, const uint16_t* w,
                           const uint16_t* table, const int64_t* indices, int64_t rows,
                           int64_t sequence, int64_t hidden, int64_t table_rows,
                           int64_t table_width, int shift_slot, int scale_slot, float eps,
                           int mode, uint16_t* out, uint16_t* resid_out, int8_t* q,
                           float* scales) {
#pragma omp parallel
  {
    float* v = (float*)malloc(sizeof(float) * (hidden > 0 ? hidden : 1));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      const int64_t tr = clampi(indices[r % sequence], table_rows);
      const uint16_t* trow = table + tr * table_width;
      for (int64_t c = 0; c < hidden; ++c) v[c] = bf2f(x[r * hidden + c]);
      if (mode == 2) {
        for (int64_t c = 0; c < hidden; ++c) {
          v[c] = rbf(v[c] + rbf(bf2f(trow[2 * hidden + c]) * bf2f(u[r * hidden + c])));
          resid_out[r * hidden + c] = f2bf(v[c]);
        }
      }
      float ms = canonical_sumsq(v, hidden) / (float)hidden;
      ms = ms + eps;
      const float rr = 1.0f / sqrtf(ms);
      for (int64_t c = 0; c < hidden; ++c) {
        const float n = rbf((v[c] * rr) * bf2f(w[c]));
        const float m = rbf(n * rbf(1.0f + bf2f(trow[(int64_t)scale_slot * hidden + c])));
        v[c] = rbf(m + bf2f(trow[(int64_t)shift_slot * hidden + c]));
      }
      if (mode == 0) {
        for (int64_t c = 0; c < hidden; ++c) out[r * hidden + c] = f2bf(v[c]);
      } else {
        quant_row_f32(v, hidden, q + r * hidden, scales + r);
      }
    }
    free(v);
  }
}

void lro_rms_adaln(const uint16_t* x, const uint16_t* w, const uint16_t* table,
                   const int64_t* indices, int64_t rows, int64_t sequence, int64_t hidden,
                   int64_t table_rows, int64_t table_width, int shift_slot, int scale_slot,
                   float eps, uint16_t* out) {
  rms_adaln_impl(x, NULL, w, table, indices, rows, sequence, hidden, table_rows, table_width,
                 shift_slot, scale_slot, eps, 0, out, NULL, NULL, NULL);
}

void lro_rms_adaln_quant(const uint16_t* x, const uint16_t* w, const uint16_t* table,
                         const int64_t* indices, int64_t rows, int64_t sequence, int64_t hidden,
                         int64_t table_rows, int64_t table_width, int shift_slot, int scale_slot,
                         float eps, int8_t* q, float* scales) {
  rms_adaln_impl(x, NULL, w, table, indices, rows, sequence, hidden, table_rows, table_width,
                 shift_slot, scale_slot, eps, 1, NULL, NULL, q, scales);
}

/* model/kernels.py:405-419: gated residual with slot 2, then slots 3/4. */
void lro_residual_rms_quant(const uint16_t* x, const uint16_t* u, const uint16_t* w,
                            const uint16_t* table, const int64_t* indices, int64_t rows,
                            int64_t sequence, int64_t hidden, int64_t table_rows,
                            int64_t table_width, float eps, uint16_t* resid_out, int8_t* q,
                            float* scales) {
  rms_adaln_impl(x, u, w, table, indices, rows, sequence, hidden, table_rows, table_width, 3, 4,
                 eps, 2, NULL, resid_out, q, scales);
}

/* Sum of squares in the canonical order, exposed for tests of the order. */
float lro_canonical_sumsq(const uint16_t* x, int64_t hidden) {
  float* v = (float*)malloc(sizeof(float) * (hidden > 0 ? hidden : 1));
  for (int64_t c = 0; c < hidden; ++c) v[c] = bf2f(x[c]);
  const float s = canonical_sumsq(v, hidden);
  free(v);
  return s;
}

/* ---------------------------------------------- QK RMSNorm + RoPE --- */
/* model/kernels.py:187-257 (_qk_norm_full_rope_paired_kernel, rotary_dim ==
 * head_dim) and :345-402 (_qk_norm_rope_kernel, rotary_dim < head_dim), as
 * called from model/fusion.py:35-52. Per (batch, token, head) row of q (and
 * of k, with its own weight):
 *   rstd = 1 / sqrt(sumsq(row) / head_dim + eps)
 *   n[d] = bf16((row[d] * rstd) * weight[d])
 *   for d < rotary_dim, half = rotary_dim / 2, c/s = bf16(cos/sin[token, d]):
 *     d <  half: out = bf16(bf16(n[d] * c) - bf16(n[d + half] * s))
 *     d >= half: out = bf16(bf16(n[d] * c) + bf16(n[d - half] * s))
 *   for d >= rotary_dim: out = n[d].
 * The sum of squares follows the reference's ordered reduction for 128-wide
 * heads (model/kernels.py:333-344, _sum128), which script/precompile.py:12-33
 * checks equal to its four-warp tl.sum: the row is cut into 32-element
 * chunks; each chunk's squares are reduced by the tree s[i] += s[i + h],
 * h = 16, ..., 1 (a warp butterfly), and the chunk sums by the same tree
 * (four chunks: (s0 + s2) + (s1 + s3)). 64- and 32-wide heads use the same
 * rule with two chunks and one. Squares of bf16 values are exact in fp32, so
 * fused or separate multiply-adds give the same sums. The reference's
 * approximate tl.rsqrt is not reproducible here; rstd = 1 / sqrt(.) instead,
 * and against the reference outputs agree to the bound that a 1-ulp change of
 * the normalized value propagates to. q/k element (b, t, h, d) is at
 * b*sequence*token_stride + t*token_stride + h*head_stride + d; outputs are
 * contiguous [batch, sequence, heads, head_dim]. */
static float qk_sumsq(const uint16_t* row, int64_t head_dim) {
  float chunk[16];
  const int64_t chunks = head_dim / 32;
  for (int64_t c = 0; c < chunks; ++c) {
    float s[32];
    for (int i = 0; i < 32; ++i) s[i] = bf2f(row[32 * c + i]) * bf2f(row[32 * c + i]);
    for (int h = 16; h >= 1; h /= 2)
      for (int i = 0; i < h; ++i) s[i] = s[i] + s[i + h];
    chunk[c] = s[0];
  }
  for (int64_t h = chunks / 2; h >= 1; h /= 2)
    for (int64_t i = 0; i < h; ++i) chunk[i] = chunk[i] + chunk[i + h];
  return chunk[0];
}

static void qk_row(const uint16_t* x, const uint16_t* w, const float* cos_row, const float* sin_row,
                   int64_t head_dim, int64_t rotary_dim, float eps, uint16_t* out) {
  float n[512];
  const float ms = qk_sumsq(x, head_dim) / (float)head_dim + eps;
  const float rstd = 1.0f / sqrtf(ms);
  for (int64_t d = 0; d < head_dim; ++d) n[d] = rbf((bf2f(x[d]) * rstd) * bf2f(w[d]));
  const int64_t half = rotary_dim / 2;
  for (int64_t d = 0; d < head_dim; ++d) {
    if (d < rotary_dim) {
      const float c = rbf(cos_row[d]), s = rbf(sin_row[d]);
      const float a = rbf(n[d] * c);
      const float b = d < half ? rbf(n[d + half] * s) : rbf(n[d - half] * s);
      out[d] = f2bf(d < half ? a - b : a + b);
    } else {
      out[d] = f2bf(n[d]);
    }
  }
}

float lro_qk_sumsq(const uint16_t* row, int64_t head_dim) { return qk_sumsq(row, head_dim); }

void lro_qk_norm_rope(const uint16_t* q, const uint16_t* k, const uint16_t* qw, const uint16_t* kw,
                      const float* cosv, const float* sinv, uint16_t* q_out, uint16_t* k_out,
                      int64_t batch, int64_t sequence, int64_t heads, int64_t q_token_stride,
                      int64_t q_head_stride, int64_t k_token_stride, int64_t k_head_stride,
                      int64_t head_dim, int64_t rotary_dim, float eps) {
  const int64_t rows = batch * sequence * heads;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t h = r % heads, t = (r / heads) % sequence, b = r / (heads * sequence);
    const uint16_t* qr = q + b * sequence * q_token_stride + t * q_token_stride + h * q_head_stride;
    const uint16_t* kr = k + b * sequence * k_token_stride + t * k_token_stride + h * k_head_stride;
    qk_row(qr, qw, cosv + t * rotary_dim, sinv + t * rotary_dim, head_dim, rotary_dim, eps,
           q_out + r * head_dim);
    qk_row(kr, kw, cosv + t * rotary_dim, sinv + t * rotary_dim, head_dim, rotary_dim, eps,
           k_out + r * head_dim);
  }
}

int lro_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------- adaLN table (GEMM) --- */
/* model/fusion.py:68-69: table = linear(F.silu(temb).to(bf16)), here from the
 * activations a = bf16(silu(temb)) [rows, k]. out[m, n] = bf16(s + bias[n]),
 * s summed in fp32 in the order defined for the gfx950 kernel: 64 lane
 * partials, lane l over 8-element chunks c = l, l + 64, ... in increasing c
 * and element order with fmaf (exact bf16 products, one rounding per step),
 * then s[i] += s[i + h] for h = 32, ..., 1. w is [n, k] row-major bf16. */
void lro_adaln_table(const uint16_t* a, const uint16_t* w, const uint16_t* bias, int64_t rows,
                     int64_t n, int64_t k, uint16_t* out) {
  const int64_t chunks = k / 8;
#pragma omp parallel for schedule(static)
  for (int64_t col = 0; col < n; ++col) {
    for (int64_t m = 0; m < rows; ++m) {
      float lane[64];
      for (int l = 0; l < 64; ++l) {
        float s = 0.0f;
        for (int64_t c = l; c < chunks; c += 64)
          for (int64_t e = 8 * c; e < 8 * c + 8; ++e)
            s = fmaf(bf2f(a[m * k + e]), bf2f(w[col * k + e]), s);
        lane[l] = s;
      }
      for (int h = 32; h >= 1; h /= 2)
        for (int i = 0; i < h; ++i) lane[i] = lane[i] + lane[i + h];
      const float b = bias ? bf2f(bias[col]) : 0.0f;
      out[m * n + col] = f2bf(lane[0] + b);
    }
  }
}
