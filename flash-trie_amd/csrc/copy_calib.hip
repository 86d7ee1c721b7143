// copy_calib.hip -- a plain device-to-device copy of known size.
//
// Reference point for the HBM counters: under rocprofv3 --pmc, FETCH_SIZE
// and WRITE_SIZE of `ftcal::copy_kernel` are compared with the bytes it is
// known to move (N read, N written per launch), which gives the scale factor
// applied to the same counters of the search kernel.  Also prints the copy
// bandwidth it reaches (HIP events).
//
// Usage: ft_copy_calib [MiB per buffer, default 1024] [launches, default 5]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace ftcal {

__global__ void __launch_bounds__(256) copy_kernel(const uint4* __restrict__ src,
                                                   uint4* __restrict__ dst,
                                                   size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = src[i];
}

__global__ void __launch_bounds__(256) fill_kernel(uint4* __restrict__ dst, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = make_uint4((uint32_t)i, 1u, 2u, 3u);
}

}  // namespace ftcal

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));            \
      return 1;                                                               \
    }                                                                         \
  } while (0)

int main(int argc, char** argv) {
  const size_t mib = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1024;
  const int launches = argc > 2 ? std::atoi(argv[2]) : 5;
  if (mib == 0 || mib > 16384 || launches < 1 || launches > 1000) {
    std::fprintf(stderr, "usage: ft_copy_calib [MiB 1..16384] [launches 1..1000]\n");
    return 2;
  }
  const size_t bytes = mib << 20;
  const size_t n = bytes / sizeof(uint4);
  uint4 *src = nullptr, *dst = nullptr;
  CHECK(hipMalloc(&src, bytes));
  CHECK(hipMalloc(&dst, bytes));
  const int grid = 256 * 8 * 4;  // 32 blocks of 256 threads per CU
  ftcal::fill_kernel<<<grid, 256>>>(src, n);
  ftcal::fill_kernel<<<grid, 256>>>(dst, n);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  double total_ms = 0.0;
  for (int i = 0; i < launches; ++i) {
    CHECK(hipEventRecord(a, 0));
    ftcal::copy_kernel<<<grid, 256>>>(src, dst, n);
    CHECK(hipEventRecord(b, 0));
    CHECK(hipEventSynchronize(b));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    total_ms += ms;
  }
  CHECK(hipGetLastError());
  const double mean_ms = total_ms / launches;
  std::printf("copy %zu MiB: read %zu B, write %zu B per launch; %d launches, "
              "mean %.3f ms, %.1f GB/s (read + write)\n",
              mib, bytes, bytes, launches, mean_ms, 2.0 * bytes / (mean_ms * 1e6));
  CHECK(hipFree(src));
  CHECK(hipFree(dst));
  return 0;
}
