// hbm_copy.hip - the practical HBM streaming ceiling of the device: a plain
// device-to-device copy of 512 MiB (16 bytes per lane, U loads in flight per
// thread, default or non-temporal cache policy), each launch timed on its own
// after a 1 GiB write has evicted the 256 MB MALL. Reports the median of 12
// launches as read + write bytes per second against the 8 TB/s peak.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e = (x);                                                            \
    if (e != hipSuccess) {                                                         \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e), __LINE__);    \
      std::exit(1);                                                                \
    }                                                                              \
  } while (0)

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// Block b copies spans of 256 * U vectors, grid-stride; every index is checked.
template <int U, bool NT>
__global__ __launch_bounds__(256) void copy_spans(const v4u* __restrict__ src, v4u* __restrict__ dst,
                                                  size_t n16) {
  const size_t span = (size_t)256 * U;
  for (size_t base = (size_t)blockIdx.x * span; base < n16; base += (size_t)gridDim.x * span) {
    v4u v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = base + (size_t)u * 256 + threadIdx.x;
      if (i < n16) v[u] = NT ? __builtin_nontemporal_load(src + i) : src[i];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = base + (size_t)u * 256 + threadIdx.x;
      if (i < n16) {
        if (NT) __builtin_nontemporal_store(v[u], dst + i);
        else dst[i] = v[u];
      }
    }
  }
}

__global__ void fill_words(unsigned* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = (unsigned)i;
}

template <int U, bool NT>
void measure(const char* name, const v4u* src, v4u* dst, size_t n16, unsigned* flush, size_t nflush,
             int grid) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  std::vector<float> ms;
  for (int r = 0; r < 12; ++r) {
    hipLaunchKernelGGL(fill_words, dim3(2048), dim3(256), 0, 0, flush, nflush);
    CHECK(hipEventRecord(a));
    hipLaunchKernelGGL((copy_spans<U, NT>), dim3(grid), dim3(256), 0, 0, src, dst, n16);
    CHECK(hipEventRecord(b));
    CHECK(hipEventSynchronize(b));
    float t = 0;
    CHECK(hipEventElapsedTime(&t, a, b));
    ms.push_back(t);
  }
  std::sort(ms.begin(), ms.end());
  const double t = ms[ms.size() / 2] * 1e-3, bytes = 2.0 * (double)n16 * 16;
  std::printf("%-22s grid %6d: %8.1f us  %6.0f GB/s  %5.1f%% of 8 TB/s\n", name, grid, t * 1e6,
              bytes / t / 1e9, bytes / t / 1e9 / 8000 * 100);
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
}

int main() {
  const size_t bytes = 512ull << 20, n16 = bytes / 16, nflush = (1ull << 30) / 4;
  v4u *src, *dst;
  unsigned* flush;
  CHECK(hipMalloc(&src, bytes));
  CHECK(hipMalloc(&dst, bytes));
  CHECK(hipMalloc(&flush, nflush * 4));
  hipLaunchKernelGGL(fill_words, dim3(2048), dim3(256), 0, 0, reinterpret_cast<unsigned*>(src), bytes / 4);
  CHECK(hipDeviceSynchronize());
  for (int grid : {4096, 32768}) {
    measure<4, false>("U4 default policy", src, dst, n16, flush, nflush, grid);
    measure<4, true>("U4 non-temporal", src, dst, n16, flush, nflush, grid);
    measure<2, true>("U2 non-temporal", src, dst, n16, flush, nflush, grid);
  }
  CHECK(hipFree(src));
  CHECK(hipFree(dst));
  CHECK(hipFree(flush));
  return 0;
}
