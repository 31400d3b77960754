// c_abi_consumer.cpp - a non-Python host of liblynnreal_amd.so.
//
// Drives the W8A8 path through the C ABI alone (include/lynnreal_amd.h):
// device buffers from the HIP runtime, the per-row quantizer
// (lr_quantize_rows, replacing model/int8.py:64-67 / model/kernels.py:8-24)
// and the INT8 GEMM with the bf16 + bias epilogue and with the raw int32
// output (lr_int8_gemm, replacing model/int8_gemm.py:96-163), then checks
// every output against a plain C++ statement of the same arithmetic:
//   s[m] = max(max_k |x[m,k]|, 1e-8) / 127 (fp32, IEEE division)
//   q = clamp(rint(x / s), -127, 127)
//   acc = sum_k q[m,k] * w[n,k] (int32, exact)
//   y = bf16(((float)acc * s[m]) * cs[n] + bias[n])   (model/int8_gemm.py:84-92)
// Compiled without FMA contraction, so the fp32 expressions round as written.
// Prints "c_abi_consumer ok ..." and exits 0 when everything is bit-exact.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "lynnreal_amd.h"

namespace {

float bf_to_f(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f_to_bf(float f) {  // round to nearest even (finite inputs)
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

#define HIP_OK(call)                                                              \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));     \
      return 2;                                                                   \
    }                                                                             \
  } while (0)

#define LR_OK_CALL(call)                                                          \
  do {                                                                            \
    int rc_ = (call);                                                             \
    if (rc_ != LR_OK) {                                                           \
      std::fprintf(stderr, "%s returned %d: %s\n", #call, rc_, lr_last_error()); \
      return 3;                                                                   \
    }                                                                             \
  } while (0)

template <typename T>
int to_device(const std::vector<T>& h, void** d) {
  HIP_OK(hipMalloc(d, h.size() * sizeof(T)));
  HIP_OK(hipMemcpy(*d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return 0;
}

template <typename T>
int to_host(const void* d, std::vector<T>& h) {
  HIP_OK(hipMemcpy(h.data(), d, h.size() * sizeof(T), hipMemcpyDeviceToHost));
  return 0;
}

int run(int M, int N, int K, uint32_t seed) {
  std::mt19937 rng(seed);
  std::normal_distribution<float> normal(0.0f, 1.0f);
  std::uniform_int_distribution<int> weight(-127, 127);
  std::uniform_real_distribution<float> scale(1e-3f, 5e-3f);

  std::vector<uint16_t> x((size_t)M * K);
  for (int m = 0; m < M; ++m)
    for (int k = 0; k < K; ++k)
      x[(size_t)m * K + k] = f_to_bf(normal(rng) * (k % 97 == 3 ? 20.0f : 1.0f));  // outlier channels
  std::vector<int8_t> w((size_t)N * K);  // [N, K] row-major: b = w^T with strides (1, K)
  for (auto& v : w) v = (int8_t)weight(rng);
  std::vector<float> cs(N);
  for (auto& v : cs) v = scale(rng);
  std::vector<uint16_t> bias(N);
  for (auto& v : bias) v = f_to_bf(0.02f * normal(rng));

  // CPU statement of the arithmetic.
  std::vector<int8_t> q_ref((size_t)M * K);
  std::vector<float> s_ref(M);
  for (int m = 0; m < M; ++m) {
    float amax = 0.0f;
    for (int k = 0; k < K; ++k) amax = std::fmax(amax, std::fabs(bf_to_f(x[(size_t)m * K + k])));
    const float s = std::fmax(amax, 1e-8f) / 127.0f;
    s_ref[m] = s;
    for (int k = 0; k < K; ++k) {
      const float v = std::rint(bf_to_f(x[(size_t)m * K + k]) / s);
      q_ref[(size_t)m * K + k] = (int8_t)std::fmin(std::fmax(v, -127.0f), 127.0f);
    }
  }
  std::vector<int32_t> acc_ref((size_t)M * N);
  std::vector<uint16_t> y_ref((size_t)M * N);
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      int32_t acc = 0;
      for (int k = 0; k < K; ++k) acc += (int32_t)q_ref[(size_t)m * K + k] * (int32_t)w[(size_t)n * K + k];
      acc_ref[(size_t)m * N + n] = acc;
      const float t = (float)acc * s_ref[m];
      const float u = t * cs[n];
      y_ref[(size_t)m * N + n] = f_to_bf(u + bf_to_f(bias[n]));
    }

  // The same through the C ABI.
  void *dx, *dw, *dcs, *dbias, *dq, *ds, *dy, *dacc;
  if (to_device(x, &dx) || to_device(w, &dw) || to_device(cs, &dcs) || to_device(bias, &dbias)) return 2;
  HIP_OK(hipMalloc(&dq, (size_t)M * K));
  HIP_OK(hipMalloc(&ds, (size_t)M * sizeof(float)));
  HIP_OK(hipMalloc(&dy, (size_t)M * N * sizeof(uint16_t)));
  HIP_OK(hipMalloc(&dacc, (size_t)M * N * sizeof(int32_t)));
  LR_OK_CALL(lr_quantize_rows(dx, M, K, (int8_t*)dq, (float*)ds, nullptr));
  LR_OK_CALL(lr_int8_gemm((const int8_t*)dq, (const int8_t*)dw, 1, K, M, N, K, (const float*)ds,
                          (const float*)dcs, dbias, dy, LR_EPI_BF16, nullptr, nullptr, 0, 0, nullptr,
                          0, 0, LR_TILE_AUTO, nullptr));
  LR_OK_CALL(lr_int8_gemm((const int8_t*)dq, (const int8_t*)dw, 1, K, M, N, K, nullptr, nullptr,
                          nullptr, dacc, LR_EPI_RAW_INT32, nullptr, nullptr, 0, 0, nullptr, 0, 0,
                          LR_TILE_AUTO, nullptr));
  HIP_OK(hipDeviceSynchronize());

  std::vector<int8_t> q((size_t)M * K);
  std::vector<float> s(M);
  std::vector<uint16_t> y((size_t)M * N);
  std::vector<int32_t> acc((size_t)M * N);
  if (to_host(dq, q) || to_host(ds, s) || to_host(dy, y) || to_host(dacc, acc)) return 2;
  for (void* p : {dx, dw, dcs, dbias, dq, ds, dy, dacc}) HIP_OK(hipFree(p));

  size_t bad_q = 0, bad_s = 0, bad_acc = 0, bad_y = 0;
  for (size_t i = 0; i < q.size(); ++i) bad_q += q[i] != q_ref[i];
  for (int m = 0; m < M; ++m) bad_s += std::memcmp(&s[m], &s_ref[m], 4) != 0;
  for (size_t i = 0; i < acc.size(); ++i) bad_acc += acc[i] != acc_ref[i];
  for (size_t i = 0; i < y.size(); ++i) bad_y += y[i] != y_ref[i];
  std::printf("M=%d N=%d K=%d: quantizer %zu/%zu and scales %zu/%d differ, int32 %zu/%zu, bf16 %zu/%zu\n", M,
              N, K, bad_q, q.size(), bad_s, M, bad_acc, acc.size(), bad_y, y.size());
  return (bad_q || bad_s || bad_acc || bad_y) ? 1 : 0;
}

}  // namespace

int main() {
  if (lr_abi_version() != LR_ABI_VERSION) {
    std::fprintf(stderr, "ABI %d, header %d\n", lr_abi_version(), LR_ABI_VERSION);
    return 4;
  }
  if (!lr_device_supported(0)) {
    std::fprintf(stderr, "device 0 is not a gfx950 GPU\n");
    return 5;
  }
  // A bad call is refused with a status and a message, before any launch.
  if (lr_int8_gemm(nullptr, nullptr, 1, 1, 4, 4, 4, nullptr, nullptr, nullptr, nullptr, 99, nullptr,
                   nullptr, 0, 0, nullptr, 0, 0, LR_TILE_AUTO, nullptr) != LR_EINVAL ||
      std::strlen(lr_last_error()) == 0) {
    std::fprintf(stderr, "invalid epilogue was not refused\n");
    return 6;
  }
  int rc = 0;
  rc |= run(300, 520, 1024, 20261201u);    // ragged M and N tiles
  rc |= run(256, 5120, 5120, 20261202u);   // benchmark config 5's M = 256 projection
  if (rc) return rc;
  std::printf("c_abi_consumer ok: quantizer, int32 and bf16 GEMM outputs bit-exact through the C ABI\n");
  return 0;
}
