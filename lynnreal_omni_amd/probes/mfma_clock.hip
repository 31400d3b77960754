// mfma_clock.hip - INT8 MFMA throughput and shader clock on gfx950 with toggling
// operands, registers only (no memory traffic). MODE 0: constant operands; 1:
// full-range random bytes re-randomised every iteration; 2: activation-like
// bytes (|a| <= 7) against full-range weights. The clock comes from s_memtime
// (shader clock) against s_memrealtime (100 MHz) over each wave.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
typedef int v4i __attribute__((ext_vector_type(4)));
#define CHECK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e), __LINE__); exit(1); } } while (0)

__device__ __forceinline__ unsigned hsh(unsigned x) { x ^= x >> 16; x *= 0x7feb352d; x ^= x >> 15; x *= 0x846ca68b; x ^= x >> 16; return x; }

template <int MODE>
__global__ __launch_bounds__(256) void mfma_data(int iters, int* out, unsigned long long* clk) {
  const unsigned long long c0 = __builtin_readcyclecounter();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  const unsigned seed = hsh(blockIdx.x * 256 + threadIdx.x);
  v4i a[4], b[8], c[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    for (int e = 0; e < 4; ++e) { unsigned v = hsh(seed + 16 * i + e); a[i][e] = MODE == 2 ? (int)(v & 0x07070707u) ^ (int)((v >> 3) & 0x80808080u) : (MODE == 0 ? 0x01020304 : (int)v); }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    for (int e = 0; e < 4; ++e) b[j][e] = MODE == 0 ? 0x05060708 : (int)hsh(seed * 7 + 16 * j + e);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) c[i][j] = v4i{0, 0, 0, 0};
#pragma unroll 1
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) c[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b[j], a[i], c[i][j], 0, 0, 0);
    if (MODE != 0) {  // new operand bits every iteration (12 VALU ops per 64 MFMAs)
      const int r = (int)hsh(it + seed);
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = (v4i){b[j].y, b[j].z, b[j].w, b[j].x ^ r};
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = MODE == 2 ? (v4i){a[i].y, a[i].z, a[i].w, a[i].x ^ (r & 0x03030303)} : (v4i){a[i].y, a[i].z, a[i].w, a[i].x ^ r};
    }
  }
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += c[i][j].x + c[i][j].y + c[i][j].z + c[i][j].w;
  if (s == 0x12345678) out[0] = s;
  if ((threadIdx.x & 63) == 0) {
    clk[(blockIdx.x * 4 + (threadIdx.x >> 6)) * 2] = __builtin_readcyclecounter() - c0;
    clk[(blockIdx.x * 4 + (threadIdx.x >> 6)) * 2 + 1] = __builtin_amdgcn_s_memrealtime() - r0;
  }
}

int main() {
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  const int blocks = cus * 2;  // 8 waves per CU, 2 per SIMD
  int* out; unsigned long long* clk;
  CHECK(hipMalloc(&out, 4));
  CHECK(hipMalloc(&clk, blocks * 4 * 2 * 8));
  unsigned long long* h = (unsigned long long*)malloc(blocks * 4 * 2 * 8);
  const int iters = 20000;
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0)); CHECK(hipEventCreate(&e1));
  for (int mode = 0; mode < 3; ++mode) {
    for (int rep = 0; rep < 2; ++rep) {
      CHECK(hipEventRecord(e0));
      if (mode == 0) hipLaunchKernelGGL(mfma_data<0>, dim3(blocks), dim3(256), 0, 0, iters, out, clk);
      else if (mode == 1) hipLaunchKernelGGL(mfma_data<1>, dim3(blocks), dim3(256), 0, 0, iters, out, clk);
      else hipLaunchKernelGGL(mfma_data<2>, dim3(blocks), dim3(256), 0, 0, iters, out, clk);
      CHECK(hipEventRecord(e1));
      CHECK(hipEventSynchronize(e1));
      float ms; CHECK(hipEventElapsedTime(&ms, e0, e1));
      CHECK(hipMemcpy(h, clk, blocks * 4 * 2 * 8, hipMemcpyDeviceToHost));
      double cyc = 0, real = 0;
      for (int w = 0; w < blocks * 4; ++w) { cyc += h[2 * w]; real += h[2 * w + 1]; }
      const double ghz = cyc / real * 0.1;
      const double ops = (double)blocks * 4 * iters * 64 * 32768.0;
      const double tops = ops / (ms * 1e-3) / 1e12;
      if (rep) printf("mode %d: %.3f ms  %.0f TOPS  sclk %.2f GHz  -> %.1f%% of peak at that clock, %.1f%% of 5000\n", mode, ms, tops, ghz,
                      100.0 * tops / (cus * 8192.0 * ghz / 1e3), tops / 50.0);
    }
  }
  return 0;
}
