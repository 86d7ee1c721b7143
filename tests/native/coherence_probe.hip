// Kernels made of coherent.h's primitives alone, compiled for gfx950 by
// tests/test_coherence_codegen.py, which checks the instructions they become.
#include "coherent.h"

using namespace ftk;

__global__ void probe_ld32(const uint32_t* p, uint32_t* o) {
  o[threadIdx.x] = ld_relaxed(p + threadIdx.x);
}
__global__ void probe_ld64(const unsigned long long* p, unsigned long long* o) {
  o[threadIdx.x] = ld_relaxed(p + threadIdx.x);
}
__global__ void probe_st32(uint32_t* p, uint32_t v) { st_dev(p + threadIdx.x, v); }
__global__ void probe_st64(unsigned long long* p, unsigned long long v) {
  st_dev(p + threadIdx.x, v);
}
// data, the wait for its stores, a barrier, then the flag: the order of a
// shared step's done word after the workgroup's pushes
__global__ void probe_signal(uint32_t* data, uint32_t* flag) {
  st_dev(data + threadIdx.x, 1u);
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) st_dev(flag, 1u);
}
