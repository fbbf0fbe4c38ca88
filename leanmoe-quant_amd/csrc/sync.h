// Hand-off of data between the workgroups of ONE launch on gfx950, for the
// fused kernels whose later phases consume what other workgroups of the same
// grid produced.
//
// The 8 XCDs each have their own L2, which is not coherent with the others.
// Data crossing workgroups inside a launch therefore moves with relaxed
// agent-scope atomic stores and loads (global_store / global_load with the
// sc1 scope bit): they are coherent across the XCDs with no L2 write-back or
// invalidate.  (The agent-scope release/acquire fences write back and
// invalidate a whole L2 each: 15.6 us per hand-off measured on MI355X with 256
// workgroups, against 0.45-1 us for the relaxed form.)  A producer
//   1. stores its results with st_coherent*,
//   2. waits for its own stores (s_waitcnt vmcnt(0)), synchronises the block,
//   3. and one lane increments a counter (relaxed agent-scope atomic add);
// a consumer polls the counters with relaxed loads until each holds the
// expected count, then reads the results with ld_coherent*.  Counters live in
// a caller-provided workspace of LEMOQ_SYNC_WORDS 32-bit words (the status
// word, then one 256-byte line per counter) and are zero between launches:
// each fused launch returns them to zero once no workgroup reads them any
// more.
//
// Every wait is bounded by a time limit measured with s_memrealtime (a
// 100 MHz clock): on expiry, or when another workgroup has already failed,
// the waiting workgroup records LEMOQ_SYNC_TIMEOUT in the status word and
// returns, so the whole grid drains.  After a failed launch the caller must
// zero the workspace again (lemoq_sync_reset).  A fused launch also needs all
// of its workgroups resident at once; the entry points check that against
// the occupancy of the kernel before launching.
#pragma once

#include "common.h"

namespace lemoq_sync {

constexpr int kLineWords = 64;  // 256 bytes per counter

__device__ __forceinline__ float ld_f32(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f32(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes as two coherent 8-byte loads / stores (p 16-byte aligned).
__device__ __forceinline__ u32x4 ld_16(const void* p) {
  uint64_t* q = reinterpret_cast<uint64_t*>(const_cast<void*>(p));
  const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (u32x4){(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

// Plain or coherent float load / store, chosen at compile time.
template <bool C>
__device__ __forceinline__ float load_f32(const float* p) {
  if constexpr (C) return ld_f32(p);
  else return *p;
}
template <bool C>
__device__ __forceinline__ void store_f32(float* p, float v) {
  if constexpr (C) st_f32(p, v);
  else *p = v;
}
template <bool C>
__device__ __forceinline__ u32x4 load_16(const void* p) {
  if constexpr (C) return ld_16(p);
  else return *reinterpret_cast<const u32x4*>(p);
}

// Wait until this wave's stores have completed (each wave calls it for its
// own stores before the block synchronises and one lane arrives).
__device__ __forceinline__ void wait_own_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void arrive(uint32_t* counter) {
  __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t now_ticks() { return __builtin_amdgcn_s_memrealtime(); }

// Called by ONE whole wave: lane i < n polls counter `first + i * kLineWords`
// until it holds at least want[i] (lane i's argument).  Returns true when every
// counter is complete; false on timeout or when the status word already
// carries a failure (it then records LEMOQ_SYNC_TIMEOUT).
__device__ __forceinline__ bool wait_counts(const uint32_t* first, int n, uint32_t want, uint32_t* status,
                                            uint64_t limit_ticks) {
  const int lane = threadIdx.x & 63;
  const uint64_t t0 = now_ticks();
  while (true) {
    bool done = true;
    if (lane < n) done = ld_u32(first + lane * kLineWords) >= want;
    if (__all(done)) return true;
    if (ld_u32(status) != 0u || now_ticks() - t0 > limit_ticks) {
      if (lane == 0) __hip_atomic_fetch_or(status, (uint32_t)LEMOQ_SYNC_TIMEOUT_BIT, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

}  // namespace lemoq_sync
