// copy_calib.hip -- calibration kernels for the search kernel's models.
//
// copy: a plain device-to-device copy of known size.  Reference point for
// the HBM counters: under rocprofv3 --pmc, FETCH_SIZE and WRITE_SIZE of
// `ftcal::copy_kernel` are compared with the bytes it is known to move (N
// read, N written per launch), which gives the scale factor applied to the
// same counters of the search kernel.  Also prints the copy bandwidth it
// reaches (HIP events).
//
// chase: the latency of one dependent global load.  One lane follows a
// pseudo-random full-period permutation of the 64-byte lines of a buffer
// (line i holds the index of the next line, (a * i + c) mod lines, a full
// cycle for a = 1 mod 4, c odd and a power-of-two line count), so every
// load's address is the previous load's value; plain loads and the
// device-coherent (agent-scope) loads the search kernel uses for shared
// data, over buffers from L2-resident to image-sized.
//
// gather: the rate of independent random loads a CU sustains.  Every lane
// of `blocks` workgroups of 1024 threads loads 8 lines at a time, each at a
// pseudo-random line of the buffer (independent addresses: up to the
// hardware's limit in flight), `rounds` times; over a buffer that the
// address translation covers and over an image-sized one; 4 bytes a lane,
// a whole 64-byte line a lane in four 16-byte loads (a cuckoo bucket read
// by one lane), or a line per four lanes.  Time per load
// and per workgroup, and the loads in flight that it implies at the chase
// latency of the same buffer size.
//
// pingpong: the latency of a device-coherent store seen by a workgroup on
// another CU (the post / claim / done handshake of a shared step): two
// workgroups pass a counter back and forth through two words, every wait
// bounded.
//
// Usage: ft_copy_calib [MiB per buffer, default 1024] [launches, default 5]
//        ft_copy_calib chase MiB [loads, default 200000]
//        ft_copy_calib gather MiB [blocks, default 1] [rounds, default 64]
//                      [0: 4 bytes a lane | 1: 64 bytes a lane | 2: 64 a quad]
//        ft_copy_calib pingpong [rounds, default 20000]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <vector>

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

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr uint64_t kLcgA = 0x5851F42D4C957F2Dull;  // = 1 mod 4
constexpr uint64_t kLcgC = 0x14057B7EF767814Full;  // odd

// line i of `lines` (a power of two) holds the next line's index
__global__ void __launch_bounds__(256) chase_init(uint32_t* buf, uint64_t lines) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < lines; i += stride)
    buf[i * 16] = (uint32_t)((kLcgA * i + kLcgC) & (lines - 1));
}

// one lane: `loads` plain then `loads` device-coherent dependent loads,
// from line out[2] on; out = {ticks plain, ticks coherent, the next line}
// (a call continues the cycle where the last one stopped: lines it has not
// touched, when the buffer holds more than the loads of all calls)
__global__ void chase_kernel(const uint32_t* buf, uint64_t loads, uint64_t* out) {
  if (threadIdx.x != 0) return;
  uint32_t idx = (uint32_t)out[2];
  const uint64_t t0 = wall_clock64();
  for (uint64_t s = 0; s < loads; ++s) idx = buf[(uint64_t)idx * 16];
  const uint64_t t1 = wall_clock64();
  for (uint64_t s = 0; s < loads; ++s) idx = ld_agent(buf + (uint64_t)idx * 16);
  const uint64_t t2 = wall_clock64();
  out[0] = t1 - t0;
  out[1] = t2 - t1;
  out[2] = idx;
}

// gather: lane l of block b, round r, load u reads line
// mix(((b * 1024 + l) * rounds + r) * 8 + u) of `lines` (a power of two):
// its first 4 bytes, or (kWhole) all 64 as four 16-byte loads, or
// (kQuad) the 16 bytes of lane l % 4 of the line of lane l - l % 4 (four
// lanes read one line together); out[b] = the block's ticks
template <int kMode>
__global__ void __launch_bounds__(1024) gather_kernel(const uint32_t* buf, uint64_t lines,
                                                      uint32_t rounds, uint64_t* out) {
  const uint64_t gl = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t gq = kMode == 2 ? (gl & ~3ull) : gl;
  uint32_t acc = 0;
  __syncthreads();
  const uint64_t t0 = wall_clock64();
  for (uint32_t r = 0; r < rounds; ++r) {
    uint32_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      uint64_t x = ((gq * rounds + r) * 8 + (uint64_t)u) * kLcgA + kLcgC;
      x ^= x >> 29;
      x *= 0xBF58476D1CE4E5B9ull;
      x ^= x >> 32;
      const uint32_t* line = buf + (x & (lines - 1)) * 16;
      if constexpr (kMode == 0) {
        v[u] = line[0];
      } else if constexpr (kMode == 1) {
        const uint4* q = (const uint4*)line;
        const uint4 a = q[0], b = q[1], c = q[2], d = q[3];
        v[u] = a.x + b.y + c.z + d.w;
      } else {
        const uint4 a = ((const uint4*)line)[gl & 3];
        v[u] = a.x + a.y + a.z + a.w;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += v[u];
  }
  __syncthreads();
  const uint64_t t1 = wall_clock64();
  if (threadIdx.x == 0) out[blockIdx.x] = t1 - t0;
  if (acc == 0x9E3779B9u) out[gridDim.x] = acc;  // keeps the loads
}

// blocks 0 and `peer` (one lane each) pass a counter: block 0 writes r to
// w[0] and waits for w[32] == r, the peer waits for w[0] == r and writes r
// to w[32]; every wait gives up after `limit` ticks.  out = {ticks, rounds
// completed}.
__global__ void pingpong_kernel(uint32_t* w, uint32_t rounds, uint32_t peer, uint64_t limit,
                                uint64_t* out) {
  if (threadIdx.x != 0 || (blockIdx.x != 0 && blockIdx.x != peer)) return;
  const bool lead = blockIdx.x == 0;
  const uint64_t t0 = wall_clock64();
  uint32_t r = 1;
  for (; r <= rounds; ++r) {
    if (lead) st_agent(w, r);
    const uint32_t* wait_on = lead ? w + 32 : w;
    const uint64_t s0 = wall_clock64();
    while (ld_agent(wait_on) != r && wall_clock64() - s0 < limit) __builtin_amdgcn_s_sleep(0);
    if (ld_agent(wait_on) != r) break;
    if (!lead) st_agent(w + 32, r);
  }
  if (lead) {
    out[0] = wall_clock64() - t0;
    out[1] = r - 1;
  }
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

static int wall_khz() {
  int khz = 0;
  (void)hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0);
  return khz > 0 ? khz : 100000;
}

static int run_chase(size_t mib, uint64_t loads) {
  if (mib == 0 || (mib & (mib - 1)) || mib > (64u << 10) || loads == 0 || loads > 10000000) {
    std::fprintf(stderr, "usage: ft_copy_calib chase MiB(power of two, <= 65536) [loads]\n");
    return 2;
  }
  const uint64_t bytes = (uint64_t)mib << 20, lines = bytes / 64;
  uint32_t* buf = nullptr;
  uint64_t* out = nullptr;
  CHECK(hipMalloc(&buf, bytes));
  CHECK(hipMalloc(&out, 3 * sizeof(uint64_t)));
  CHECK(hipMemset(out, 0, 3 * sizeof(uint64_t)));
  ftcal::chase_init<<<256 * 8, 256>>>(buf, lines);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  uint64_t h[3] = {0, 0, 0};
  // the first call warms the code path; the second goes on along the cycle
  // (lines not touched yet unless the buffer holds fewer than 4 x loads)
  for (int pass = 0; pass < 2; ++pass) {
    ftcal::chase_kernel<<<1, 64>>>(buf, loads, out);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(h, out, sizeof(h), hipMemcpyDeviceToHost));
  }
  const double ns_tick = 1e6 / wall_khz();
  std::printf("chase %zu MiB (%llu lines), %llu dependent loads%s: plain %.1f ns, "
              "device-coherent %.1f ns per load\n",
              mib, (unsigned long long)lines, (unsigned long long)loads,
              lines >= 4 * loads ? " on lines not touched before" : " (revisiting lines)",
              h[0] * ns_tick / loads, h[1] * ns_tick / loads);
  CHECK(hipFree(buf));
  CHECK(hipFree(out));
  return 0;
}

static int run_gather(size_t mib, uint32_t blocks, uint32_t rounds, int mode) {
  if (mode < 0 || mode > 2 || mib == 0 || (mib & (mib - 1)) || mib > (64u << 10) || blocks == 0 || blocks > 4096 ||
      rounds == 0 || rounds > 4096) {
    std::fprintf(stderr, "usage: ft_copy_calib gather MiB(power of two, <= 65536) "
                         "[blocks <= 4096] [rounds <= 4096]\n");
    return 2;
  }
  const uint64_t bytes = (uint64_t)mib << 20, lines = bytes / 64;
  uint32_t* buf = nullptr;
  uint64_t* out = nullptr;
  CHECK(hipMalloc(&buf, bytes));
  CHECK(hipMalloc(&out, (blocks + 1) * sizeof(uint64_t)));
  ftcal::chase_init<<<256 * 8, 256>>>(buf, lines);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  const double ns_tick = 1e6 / wall_khz();
  std::vector<uint64_t> h(blocks + 1);
  for (int pass = 0; pass < 2; ++pass) {
    if (mode == 0) ftcal::gather_kernel<0><<<blocks, 1024>>>(buf, lines, rounds, out);
    else if (mode == 1) ftcal::gather_kernel<1><<<blocks, 1024>>>(buf, lines, rounds, out);
    else ftcal::gather_kernel<2><<<blocks, 1024>>>(buf, lines, rounds, out);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(h.data(), out, (blocks + 1) * sizeof(uint64_t), hipMemcpyDeviceToHost));
  }
  uint64_t mx = 0, sum = 0;
  for (uint32_t b = 0; b < blocks; ++b) {
    mx = std::max(mx, h[b]);
    sum += h[b];
  }
  const double per_wg = 1024.0 * 8 * rounds;
  static const char* kHow[3] = {"4 bytes a lane", "64 bytes a lane as 4 x 16",
                                "64 bytes per 4 lanes, 16 each"};
  std::printf("gather (%s) %zu MiB, %u workgroup(s) x 1024 lanes x %u rounds x 8 loads: "
              "%.2f ns per load per workgroup (mean), %.2f (slowest); %.2f loads per ns "
              "over the device\n",
              kHow[mode], mib, blocks, rounds, sum * ns_tick / blocks / per_wg, mx * ns_tick / per_wg,
              per_wg * blocks / (mx * ns_tick));
  CHECK(hipFree(buf));
  CHECK(hipFree(out));
  return 0;
}

static int run_pingpong(uint32_t rounds) {
  if (rounds == 0 || rounds > 1000000) {
    std::fprintf(stderr, "usage: ft_copy_calib pingpong [rounds <= 1000000]\n");
    return 2;
  }
  uint32_t* w = nullptr;
  uint64_t* out = nullptr;
  CHECK(hipMalloc(&w, 256));
  CHECK(hipMalloc(&out, 2 * sizeof(uint64_t)));
  const double ns_tick = 1e6 / wall_khz();
  // the dispatcher deals blocks to the 8 XCDs in turn: block 8 shares block
  // 0's XCD, block 1 is on the next one
  for (uint32_t peer : {8u, 1u}) {
    CHECK(hipMemset(w, 0, 256));
    ftcal::pingpong_kernel<<<16, 64>>>(w, rounds, peer, 10000000ull, out);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    uint64_t h[2] = {0, 0};
    CHECK(hipMemcpy(h, out, sizeof(h), hipMemcpyDeviceToHost));
    std::printf("pingpong with block %u (%s XCD): %llu of %u rounds, %.1f ns one way\n", peer,
                peer == 8 ? "same" : "another", (unsigned long long)h[1], rounds,
                h[1] ? h[0] * ns_tick / (2.0 * h[1]) : 0.0);
  }
  CHECK(hipFree(w));
  CHECK(hipFree(out));
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && std::strcmp(argv[1], "chase") == 0)
    return run_chase(argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 0,
                     argc > 3 ? std::strtoull(argv[3], nullptr, 10) : 200000);
  if (argc > 1 && std::strcmp(argv[1], "gather") == 0)
    return run_gather(argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 0,
                      argc > 3 ? (uint32_t)std::strtoul(argv[3], nullptr, 10) : 1u,
                      argc > 4 ? (uint32_t)std::strtoul(argv[4], nullptr, 10) : 64u,
                      argc > 5 ? std::atoi(argv[5]) : 0);
  if (argc > 1 && std::strcmp(argv[1], "pingpong") == 0)
    return run_pingpong(argc > 2 ? (uint32_t)std::strtoul(argv[2], nullptr, 10) : 20000);
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
