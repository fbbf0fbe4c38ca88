// HBM read-bandwidth probe: streams a buffer once with 16-byte nontemporal
// loads and folds it into one dword per block, so nothing but the read is
// timed.  Used as the roofline denominator ("measured read bandwidth") and,
// over a buffer larger than the 256 MB Infinity Cache, to evict the caches
// before a cold kernel timing.  It restates the method of the reference's
// bandwidth probe (tools/probe_machine.py:392-505: a large read-reduce), not
// its code.
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void read_probe_kernel(const u32x4* __restrict__ src,
                                                         int64_t n16, uint32_t* __restrict__ out) {
  uint32_t a = 0u;
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  // Four independent loads in flight per lane per iteration.
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 v0 = __builtin_nontemporal_load(src + i);
    const u32x4 v1 = __builtin_nontemporal_load(src + i + stride);
    const u32x4 v2 = __builtin_nontemporal_load(src + i + 2 * stride);
    const u32x4 v3 = __builtin_nontemporal_load(src + i + 3 * stride);
    a ^= (v0.x + v0.y + v0.z + v0.w) ^ (v1.x + v1.y + v1.z + v1.w) ^
         (v2.x + v2.y + v2.z + v2.w) ^ (v3.x + v3.y + v3.z + v3.w);
  }
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    a ^= v.x + v.y + v.z + v.w;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) a ^= (uint32_t)__shfl_xor((int)a, o, 64);
  __shared__ uint32_t red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// Plain copy with 16-byte loads and stores: each byte is read once and
// written once, so its profiler counters calibrate FETCH_SIZE / WRITE_SIZE.
__global__ __launch_bounds__(256) void copy_probe_kernel(const u32x4* __restrict__ src,
                                                         u32x4* __restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
    dst[i] = __builtin_nontemporal_load(src + i);
}

}  // namespace

extern "C" int lemoq_read_probe(const void* src, int64_t n_bytes, uint32_t* out, int64_t blocks,
                                void* stream) {
  if (!src || !out) return LEMOQ_ERR_NULL;
  if (n_bytes <= 0 || n_bytes % 16 != 0 || blocks <= 0 || blocks > 65536) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(src)) return LEMOQ_ERR_ALIGN;
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, lemoq_stream(stream),
                     reinterpret_cast<const u32x4*>(src), n_bytes / 16, out);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_copy_probe(const void* src, void* dst, int64_t n_bytes, int64_t blocks,
                                void* stream) {
  if (!src || !dst) return LEMOQ_ERR_NULL;
  if (n_bytes <= 0 || n_bytes % 16 != 0 || blocks <= 0 || blocks > 65536) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(src) || !lemoq_aligned16(dst)) return LEMOQ_ERR_ALIGN;
  const char* s = static_cast<const char*>(src);
  const char* d = static_cast<const char*>(dst);
  if (s < d + n_bytes && d < s + n_bytes) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(copy_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, lemoq_stream(stream),
                     reinterpret_cast<const u32x4*>(src), reinterpret_cast<u32x4*>(dst), n_bytes / 16);
  LEMOQ_CHECK_LAUNCH();
}
