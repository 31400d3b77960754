/*
 * lynnreal_amd.h - C ABI of the MI355X (gfx950) W8A8 DiT projection path.
 *
 * The reference (LynnReal-Omni) exposes this path as Python functions that
 * launch Triton kernels; it has no FFI. Each entry point below replaces one
 * of those functions and cites it (paths relative to the reference checkout).
 * The Python host layer in lynnreal_omni_amd/ keeps the reference's Python
 * signatures and calls these entry points through ctypes (the integer-argument
 * ones through a CPython fast-call shim); tests/abi_host/c_abi_consumer.cpp is
 * a C++ host that uses them directly.
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are raw device pointers. bf16 tensors are passed as
 *     `const void*` / `void*` and hold IEEE bfloat16 bit patterns.
 *   - Tensors are dense and row-major unless a stride argument says otherwise.
 *   - The library never allocates or frees device memory: the caller owns
 *     every input and output buffer (the reference allocates outputs with
 *     torch.empty on the input's device, kernels.py:21-22, int8_gemm.py:134).
 *   - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued
 *     on it with no host synchronisation.
 *   - Every entry point returns an LR_* status. On failure lr_last_error()
 *     returns a message for the calling thread.
 *   - `indices` index rows of an adaLN table. Values outside [0, table_rows)
 *     are clamped into that range so that a bad index can never read outside
 *     the table (the reference performs no check).
 */
#ifndef LYNNREAL_AMD_H
#define LYNNREAL_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LR_ABI_VERSION 1

/* Status codes. The Python layer maps them to exceptions:
 * EINVAL -> ValueError, EUNSUPPORTED -> RuntimeError("... not supported"),
 * ENOMEM -> torch.cuda.OutOfMemoryError, EHIP -> RuntimeError. */
#define LR_OK 0
#define LR_EINVAL 1
#define LR_EUNSUPPORTED 2
#define LR_EHIP 3
#define LR_ENOMEM 4

/* GEMM epilogues (lr_int8_gemm `epilogue`). */
#define LR_EPI_BF16 0           /* bf16(((float)acc*row_scale)*col_scale + bias)      */
#define LR_EPI_GELU_TANH 1      /* bf16(gelu_tanh(y)), y = the LR_EPI_BF16 value       */
#define LR_EPI_GATED_RESIDUAL 2 /* bf16(x + bf16(gate*y)), y = the LR_EPI_BF16 value   */
#define LR_EPI_RAW_INT32 3      /* int32 accumulators, no scaling                      */

/* GEMM tile configurations (lr_int8_gemm `tile`). */
#define LR_TILE_AUTO 0
#define LR_TILE_256x256 1
#define LR_TILE_256x128 2
#define LR_TILE_128x256 3
#define LR_TILE_128x128 4
#define LR_TILE_64x128 5
#define LR_TILE_GENERIC 6 /* any strides / K; slow, used when the fast path cannot run */
#define LR_TILE_256x256_W4x2 7 /* 256x256 with a 4x2 wave grid (64x128 per wave) */
#define LR_TILE_256x192 8 /* 256x192 with a 4x2 wave grid (64x96 per wave) */
#define LR_TILE_256x80 9 /* 256x80, 4 waves of 64x80: weight streaming for M <= 256 */
#define LR_TILE_64x80 10 /* 64x80, 4 waves of 16x80: weight streaming for M <= 256 */
#define LR_TILE_128x160 11 /* 128x160, 4 waves of 64x80: weight streaming for M <= 256 */
#define LR_TILE_192x256 12 /* 192x256, 8 waves of 96x64: fills the last wave of tiles at long K */
#define LR_TILE_256x256_PERSISTENT 13 /* 256x256 on a persistent grid (one workgroup per CU looping
                                        over the tiles, each tile's last k-steps loading the next
                                        tile's first ones); replaces model/int8_tma.py:12-41 */

/* Library version; bumped whenever a signature below changes. */
int lr_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* lr_last_error(void);

/* 1 if `device` is a gfx950 GPU this library was built for, else 0.
 * Replaces the capability gate of model/acceleration.py:5-18. */
int lr_device_supported(int device);

/* Per-row symmetric INT8 quantizer.
 * Replaces model/kernels.py:19-24 (quantize_rows) with the arithmetic of the
 * torch path model/int8.py:66-67:
 *   s[r] = max(max_c |x[r,c]|, 1e-8f) / 127.0f
 *   q[r,c] = clamp(rint_half_even(x[r,c] / s[r]), -127, 127)
 * x bf16 [rows, width]; q int8 [rows, width]; scales fp32 [rows]. */
int lr_quantize_rows(const void* x, int64_t rows, int64_t width, int8_t* q, float* scales,
                     void* stream);

/* Element types of lr_quantize_rows_typed. */
#define LR_DTYPE_BF16 0
#define LR_DTYPE_F16 1
#define LR_DTYPE_F32 2

/* lr_quantize_rows for bf16, fp16 or fp32 rows x (LR_DTYPE_*): the
 * reference's Triton quantizer loads any float row as fp32
 * (model/kernels.py:8-16); the scale and the IEEE quotient x / s are the
 * same as for bf16 rows. */
int lr_quantize_rows_typed(const void* x, int dtype, int64_t rows, int64_t width, int8_t* q,
                           float* scales, void* stream);

/* INT8 x INT8 -> INT32 GEMM with a fused epilogue.
 * Replaces model/int8_gemm.py:96-163 (int8_matmul) and its Triton kernel
 * model/int8_gemm.py:13-46:
 *   acc[m,n] = sum_k A[m,k] * B[k,n]                  (exact int32)
 *   y[m,n]   = bf16(((float)acc * row_scale[m]) * col_scale[n] + bias[n])
 * A int8 [M,K] row-major. B int8 with B[k,n] at b[k*b_stride_k + n*b_stride_n];
 * the weight layout of Int8Linear (a [K,N] view of [N,K] storage) has
 * b_stride_k = 1, b_stride_n = K and takes the MFMA fast path.
 * row_scale fp32 [M]; col_scale fp32 [N]; bias bf16 [N] or NULL.
 * c: bf16 [M,N] (or int32 [M,N] for LR_EPI_RAW_INT32).
 * Gated residual (LR_EPI_GATED_RESIDUAL; model/kernels.py:131-153 applied to
 * the GEMM output): residual bf16 [M,N], table bf16 [table_rows, table_width],
 * indices int64 [sequence]; row m uses table row indices[m % sequence] and
 * gate = table[row, gate_slot*N + n]. Unused arguments may be NULL/0.
 * tile: LR_TILE_* (LR_TILE_AUTO picks by shape). */
int lr_int8_gemm(const int8_t* a, const int8_t* b, int64_t b_stride_k, int64_t b_stride_n,
                 int64_t m, int64_t n, int64_t k, const float* row_scale, const float* col_scale,
                 const void* bias, void* c, int epilogue, const void* residual, const void* table,
                 int64_t table_rows, int64_t table_width, const int64_t* indices,
                 int64_t sequence, int gate_slot, int tile, void* stream);

/* lr_int8_gemm with a caller-provided device workspace for split-K: the
 * K dimension is divided over `splits` workgroups per output tile, which
 * write int32 partial sums to the workspace; a second kernel adds them (exact
 * integer sums) and applies the same epilogue, so the outputs equal
 * lr_int8_gemm's bit for bit. splits: 0 = chosen by shape (split only where
 * the tiles would leave CUs idle), 1 = none, 2..64 = forced (K % 128 == 0,
 * splits <= K / 128, N % 4 == 0). The library never allocates: workspace is
 * device memory of workspace_bytes >= lr_int8_gemm_workspace_size (256-byte
 * aligned), used only by the call's kernels on `stream`, so calls that share
 * one workspace must be ordered on one stream. With workspace NULL no split
 * is taken unless forced (then LR_EINVAL). Replaces the same reference
 * functions as lr_int8_gemm (model/int8_gemm.py:96-163, :13-46), whose Triton
 * autotuner covers small M with small tiles (model/int8_gemm.py:49-52). */
int lr_int8_gemm_ws(const int8_t* a, const int8_t* b, int64_t b_stride_k, int64_t b_stride_n,
                    int64_t m, int64_t n, int64_t k, const float* row_scale, const float* col_scale,
                    const void* bias, void* c, int epilogue, const void* residual, const void* table,
                    int64_t table_rows, int64_t table_width, const int64_t* indices,
                    int64_t sequence, int gate_slot, void* workspace, int64_t workspace_bytes,
                    int splits, int tile, void* stream);

/* Workspace bytes lr_int8_gemm_ws needs for this shape, splits and tile
 * (0 when its schedule does not split K). Sizing helper of lr_int8_gemm_ws;
 * the reference has no counterpart (its Triton GEMM keeps no partials). */
int64_t lr_int8_gemm_workspace_size(int64_t m, int64_t n, int64_t k, int splits, int tile);

/* lr_int8_gemm_ws without the workspace: the split-K slices go to a
 * file-scope device array of the library (32 MiB, one per GPU, held until
 * the process ends), so the call allocates nothing and takes no workspace.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). A split whose slices need more than 32 MiB is refused with
 * LR_EINVAL (the automatic choice needs at most about 21 MiB); calls that
 * overlap on one GPU share the array and race. Same arguments, arithmetic
 * and outputs as lr_int8_gemm_ws. */
int lr_int8_gemm_noalloc(const int8_t* a, const int8_t* b, int64_t b_stride_k, int64_t b_stride_n,
                         int64_t m, int64_t n, int64_t k, const float* row_scale,
                         const float* col_scale, const void* bias, void* c, int epilogue,
                         const void* residual, const void* table, int64_t table_rows,
                         int64_t table_width, const int64_t* indices, int64_t sequence,
                         int gate_slot, int splits, int tile, void* stream);

/* Stand-alone INT32 -> bf16 dequant epilogue.
 * Replaces model/kernels.py:41-46 (int8_epilogue):
 *   out[m,n] = bf16(((float)acc[m,n] * a_scale[m]) * w_scale[n] + bias[n]).
 * acc int32 [M,N]; a_scale fp32 [M]; w_scale fp32 [N]; bias bf16 [N] or NULL. */
int lr_int8_epilogue(const int32_t* acc, const float* a_scale, const float* w_scale,
                     const void* bias, void* out, int64_t m, int64_t n, void* stream);

/* Fused RMSNorm + adaLN modulate, bf16 out.
 * Replaces model/kernels.py:260-272 (_rms_adaln) / kernel :48-78. Row r uses
 * token r % sequence and table row tr = indices[token]:
 *   ss = sum_c x^2 (fp32, fixed order: see lr_rms_adaln_quant)
 *   rr = 1 / sqrt(ss / hidden + eps)
 *   n  = bf16((x * rr) * weight[c])
 *   y  = bf16(bf16(n * bf16(1 + table[tr, scale_slot*hidden + c]))
 *             + table[tr, shift_slot*hidden + c])
 * x bf16 [rows, hidden]; weight bf16 [hidden]; out bf16 [rows, hidden]. */
int lr_rms_adaln(const void* x, const void* weight, const void* table, const int64_t* indices,
                 void* out, int64_t rows, int64_t sequence, int64_t hidden, int64_t table_rows,
                 int64_t table_width, int shift_slot, int scale_slot, float eps, void* stream);

/* Fused RMSNorm + adaLN modulate + per-row INT8 quantization.
 * Replaces model/kernels.py:275-289 (_rms_adaln_quant_int8) / kernel :81-128.
 * y as in lr_rms_adaln, then q/scales as in lr_quantize_rows.
 * The sum of squares has one defined order so that results are reproducible:
 * the row is cut into 8-element chunks; chunk j is accumulated into slot
 * j % 256 (chunks in increasing j, elements in order, s = fma(x, x, s) in
 * fp32); the 256 slots are then combined by s[i] += s[i + h] for
 * h = 128, 64, ..., 1. */
int lr_rms_adaln_quant(const void* x, const void* weight, const void* table,
                       const int64_t* indices, int8_t* q, float* scales, int64_t rows,
                       int64_t sequence, int64_t hidden, int64_t table_rows, int64_t table_width,
                       int shift_slot, int scale_slot, float eps, void* stream);

/* Gated residual + RMSNorm + adaLN modulate + INT8 quantization.
 * Replaces model/kernels.py:405-419 (residual_rms_quant; branch :101-105):
 *   x' = bf16(x + bf16(table[tr, 2*hidden + c] * u)), stored to residual_out,
 * then lr_rms_adaln_quant on x' with shift slot 3 and scale slot 4. */
int lr_residual_rms_quant(const void* x, const void* update, const void* weight,
                          const void* table, const int64_t* indices, void* residual_out,
                          int8_t* q, float* scales, int64_t rows, int64_t sequence,
                          int64_t hidden, int64_t table_rows, int64_t table_width, float eps,
                          void* stream);

/* Gated residual. Replaces model/kernels.py:292-304 (_gated_residual) /
 * kernel :131-153:  out = bf16(x + bf16(table[tr, gate_slot*hidden + c] * u)).
 * x, u, out bf16 [rows, hidden]. */
int lr_gated_residual(const void* x, const void* update, const void* table,
                      const int64_t* indices, void* out, int64_t rows, int64_t sequence,
                      int64_t hidden, int64_t table_rows, int64_t table_width, int gate_slot,
                      void* stream);

/* SwiGLU. Replaces model/kernels.py:307-315 (_swiglu) / kernel :156-166:
 *   out[r,c] = bf16(v * bf16(g * sigmoid(g))), v = p[r,c], g = p[r,inner+c].
 * p bf16 [rows, 2*inner]; out bf16 [rows, inner]. */
int lr_swiglu(const void* p, void* out, int64_t rows, int64_t inner, void* stream);

/* SwiGLU + INT8 quantization. Replaces model/kernels.py:318-328
 * (_swiglu_quant_int8) / kernel :169-185:
 *   a = bf16(v * bf16(g * sigmoid(g))), then q/scales as lr_quantize_rows.
 * q int8 [rows, inner]; scales fp32 [rows]. */
int lr_swiglu_quant(const void* p, int8_t* q, float* scales, int64_t rows, int64_t inner,
                    void* stream);

/* Element-wise GELU (tanh approximation), bf16 in and out:
 *   out = bf16(0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))).
 * The reference has no in-tree kernel for it; its only GELU-tanh INT8 path is
 * comfy-kitchen's int8_linear(input_act="gelu_tanh"), exercised at
 * comfyui/custom_nodes/ComfyUI-LynnReal/tools/verify_sampling_safety.py:59. */
int lr_gelu_tanh(const void* x, void* out, int64_t count, void* stream);

/* GELU-tanh fused with the per-row INT8 quantizer, the FFN re-quantization of
 * a GELU-tanh FFN: a = bf16(gelu_tanh(x)) as lr_gelu_tanh computes it, then
 * q/scales as lr_quantize_rows. The GELU counterpart of lr_swiglu_quant
 * (model/kernels.py:318-328, which fuses the reference's FFN activation into
 * its re-quantizer); equal bit for bit to lr_gelu_tanh followed by
 * lr_quantize_rows. x bf16 [rows, width]; q int8 [rows, width]; scales fp32
 * [rows]. */
int lr_gelu_quant(const void* x, int8_t* q, float* scales, int64_t rows, int64_t width,
                  void* stream);

/* Per-head RMSNorm of Q and K fused with rotary embedding. Replaces the
 * launches at model/fusion.py:35-52 of model/kernels.py:187-257
 * (_qk_norm_full_rope_paired_kernel, rotary_dim == head_dim) and :345-402
 * (_qk_norm_rope_kernel, rotary_dim < head_dim). Per (batch, token, head)
 * row of q (k likewise with k_weight):
 *   rstd = 1 / sqrt(sumsq(row) / head_dim + eps), n = bf16((row * rstd) * w)
 *   d <  rotary_dim/2: out = bf16(bf16(n[d]*c[d]) - bf16(n[d + rotary_dim/2]*s[d]))
 *   d <  rotary_dim:   out = bf16(bf16(n[d]*c[d]) + bf16(n[d - rotary_dim/2]*s[d]))
 *   d >= rotary_dim:   out = n[d]
 * with c, s = bf16(cos/sin[token, d]) from fp32 [sequence, rotary_dim]. The
 * sum of squares follows model/kernels.py:333-344 (_sum128): 32-element
 * chunks, each reduced by s[i] += s[i + h], h = 16 .. 1, then the chunk sums
 * by the same tree ((s0 + s2) + (s1 + s3) for 128-wide heads). q/k element
 * (b, t, h, d) is at b*sequence*token_stride + t*token_stride + h*head_stride
 * + d (bf16 elements); q_out/k_out are contiguous [batch, sequence, heads,
 * head_dim]. head_dim in {32, 64, 128}; rotary_dim a multiple of 16 (0 included). */
int lr_qk_norm_rope(const void* q, const void* k, const void* q_weight, const void* k_weight,
                    const float* cos, const float* sin, void* q_out, void* k_out, int64_t batch,
                    int64_t sequence, int64_t heads, int64_t q_token_stride, int64_t q_head_stride,
                    int64_t k_token_stride, int64_t k_head_stride, int64_t head_dim,
                    int64_t rotary_dim, float eps, void* stream);

/* Row gather. Replaces the index_select calls of Flash token selection at
 * model/flash.py:71-80 (compress: hidden.index_select(1, keep),
 * indices.index_select(0, keep), rotary value.index_select(-2, keep),
 * mask.index_select(-1, keep)):
 *   dst[o, i, :] = src[o, index[i], :],  o < outer, i < dst_rows,
 * src [outer, src_rows, row_bytes], dst [outer, dst_rows, row_bytes], any
 * element type (rows are bytes). Indices must lie in [0, src_rows); others
 * are clamped into it. */
int lr_gather_rows(const void* src, const int64_t* index, void* dst, int64_t outer,
                   int64_t src_rows, int64_t dst_rows, int64_t row_bytes, void* stream);

/* Flash residual restore. Replaces model/flash.py:82-85 (restore):
 *   out[o, t, c] = bf16(full[o, t, c]
 *                       + bf16(bf16(current - input)[o, inverse[t], c] * gain))
 * full, out bf16 [outer, rows, width]; current, input bf16 [outer,
 * compressed_rows, width]; inverse int64 [rows] in [0, compressed_rows)
 * (others are clamped). out may alias full. */
int lr_flash_restore(const void* full, const void* current, const void* input,
                     const int64_t* inverse, void* out, int64_t outer, int64_t rows,
                     int64_t compressed_rows, int64_t width, float gain, void* stream);

/* Nearest-anchor map of Flash token selection. Replaces the search loop of
 * model/flash.py:26-32 (torch.cdist + argmin per 1024 dropped rows): for each
 * dropped row d, among anchor rows a with positions[a, 0] == positions[d, 0],
 * the first a of least (h_d - h_a)^2 + (w_d - w_a)^2 (fp32 coordinates,
 * distance in fp64; no such anchor gives the first anchor), then
 *   inverse[dropped[i]] = inverse[anchors[a]].
 * positions fp32 [tokens, 3] (time, h, w); dropped, anchors int64 row numbers
 * in [0, tokens) (others are clamped); inverse int64 [tokens], updated in
 * place at the dropped rows. */
int lr_flash_nearest_anchor(const float* positions, int64_t tokens, const int64_t* dropped,
                            int64_t n_dropped, const int64_t* anchors, int64_t n_anchors,
                            int64_t* inverse, void* stream);

/* adaLN modulation table. Replaces model/fusion.py:68-69 (and
 * elementwise_fusion.py:8-10): linear(F.silu(temb).to(bf16)), a skinny bf16
 * GEMM over the time embeddings:
 *   a = bf16(silu(temb)) (silu(x) = x / (1 + exp(-x)) in fp32; bf16(temb)
 *       when apply_silu is 0)
 *   out[m, n] = bf16(sum_k a[m, k] * weight[n, k] + bias[n])
 * with the fp32 sum in a fixed order: 64 partials, partial l over the
 * 8-element chunks c = l, l + 64, ... (fma, element order), combined by
 * s[i] += s[i + h], h = 32 .. 1. temb fp32 or bf16 [rows, in_features];
 * weight bf16 [out_features, in_features] (nn.Linear layout); bias bf16
 * [out_features] or NULL; out bf16 [rows, out_features]. in_features a
 * multiple of 8, at most 8192. */
int lr_adaln_table(const void* temb, int temb_is_bf16, int apply_silu, const void* weight,
                   const void* bias, void* out, int64_t rows, int64_t in_features,
                   int64_t out_features, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LYNNREAL_AMD_H */
