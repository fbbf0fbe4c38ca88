// HBM read-bandwidth probe: streams a buffer once with 16-byte nontemporal
// loads and folds it into one dword per block, so nothing but the read is
// timed.  Used as the roofline denominator ("measured read bandwidth") and,
// over a buffer larger than the 256 MB Infinity Cache, to evict the caches
// before a cold kernel timing.  It restates the method of the reference's
// bandwidth probe (tools/probe_machine.py:392-505: a large read-reduce), not
// its code.
#include "common.h"

namespace {

// Block b reads the contiguous elements [b*per16, min((b+1)*per16, n16)) of
// the buffer (per16 a multiple of 256, i.e. 4 KB); wave w of the block reads
// its 4 KB chunks w, w+4, ... with four 1 KB loads in flight (addresses
// clamped into the block's range, the excess masked).  One contiguous 4 KB
// chunk per wave over a grid of 16 KB blocks is the fastest read pattern
// measured on this GPU (about 7.1 TB/s over 1 GiB, against 6.2 TB/s for a
// grid-stride walk).
__global__ __launch_bounds__(256) void read_probe_kernel(const u32x4* __restrict__ src,
                                                         int64_t n16, int64_t per16,
                                                         uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t b0 = (int64_t)blockIdx.x * per16;
  const int64_t b1 = b0 + per16 < n16 ? b0 + per16 : n16;
  uint32_t a = 0u;
  for (int64_t c = b0 + (int64_t)wave * 256; c < b1; c += 4 * 256) {
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t k = c + j * 64 + lane;
      v[j] = __builtin_nontemporal_load(src + (k < b1 ? k : b1 - 1));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c + j * 64 + lane < b1) a ^= v[j].x + v[j].y + v[j].z + v[j].w;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) a ^= (uint32_t)__shfl_xor((int)a, o, 64);
  __shared__ uint32_t red[4];
  if (lane == 0) red[wave] = a;
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
  const int64_t n16 = n_bytes / 16;
  int64_t per16 = (n16 + blocks - 1) / blocks;
  per16 = (per16 + 255) / 256 * 256;  // whole 4 KB chunks per block
  const int64_t grid = (n16 + per16 - 1) / per16;  // blocks beyond the data read nothing
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)grid), dim3(256), 0, lemoq_stream(stream),
                     reinterpret_cast<const u32x4*>(src), n16, per16, out);
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
