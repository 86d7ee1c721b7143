// coherent.h -- the loads and stores through which a request's workgroups
// share data during a search (tbs_kernel.hip), and the wait between a
// writer's data and its signal.
//
// A writer stores shared data with st_dev, waits for the stores
// (wait_stores), then signals with st_dev; a reader loads the signal with
// ld_relaxed and, once it has seen it, the data.  What this rests on is the
// code LLVM generates for gfx942-class targets
// (gfx950 included) from monotonic agent-scope atomics -- the "Memory Model
// GFX942" table of LLVM's AMDGPUUsage: a load is `global_load ... sc1`, a
// store `global_store ... sc1`, each served at the coherence point of the
// agent rather than from a possibly stale non-coherent line; and on the
// ordering the hardware gives a wave: memory operations issue in program
// order, `s_waitcnt vmcnt(0)` returns only once every earlier store has
// been acknowledged, and no load after a branch on a loaded value issues
// before that value is back.  Under the C++ memory model alone relaxed
// atomics would not order the data against the flag; release / acquire
// would, but their agent-scope form writes back / invalidates the L2 of the
// XCD (buffer_wbl2 sc1 / buffer_inv sc1), which measured ~50% of step-1
// time when every helper did it every step.  The inline `s_waitcnt` below
// carries a memory clobber, so the compiler keeps the stores before it.
//
// tests/test_coherence_codegen.py compiles these primitives for gfx950 and
// checks the instructions they become.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ftk {

__device__ __forceinline__ unsigned long long ld_relaxed(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_relaxed(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this wave's stores are complete (acknowledged at device
// scope); the memory clobber keeps the compiler from moving them past it.
__device__ __forceinline__ void wait_stores() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

}  // namespace ftk
