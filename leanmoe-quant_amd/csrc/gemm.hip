// Batched (prefill) GEMM on the gfx950 matrix cores: Y = X W^T with X (M, K)
// fp16 and W (N, K) either w8 (int8 codes + fp16 scales per group of 128
// along K) or fp16, fp32 accumulation.
//
// The w8 path dequantises W exactly as the reference's separate path does
// before its F.linear (QuantLinear.forward for T > 1, src/lemoq/quant/
// linear.py:365-395, 471-480): w = fp16(code * scale_fp16) -- the exact
// code, converted to fp16, times the fp16 scale in one fp16 rounding
// (v_pk_mul_f16).
//
// Tiling: 4 waves per block (2 x 2), block tiles of 128 x 128, or 64 x 128
// when a grid of 128 x 128 tiles would leave compute units idle; the stage
// pipeline of gemm_core.h.  Tiles are numbered n-major (consecutive tiles
// share the weight tile) and each XCD takes a contiguous range of them.
//
// Rows: X row m may be gathered (x_rows[m]); the output is fp16 rows with an
// optional fp16 residual added in one rounding (torch's fp16 add).  Rows and
// columns beyond M/N are clamped on load and not stored.  When the output
// (and residual) rows are 16-byte aligned, the block stages its fp16 tile in
// LDS and writes whole row segments in 16-byte chunks; otherwise each lane
// stores its own elements.
#include "gemm_core.h"

#include <mutex>

namespace {

using namespace lemoq_gemm;

struct GemmArgs {
  const uint16_t* x;       // (rows, x_ld) fp16
  int64_t x_ld;
  const int32_t* x_rows;   // optional gather (M)
  int64_t M, N, K;
  const int8_t* codes;     // w8: (N, K) int8
  const uint16_t* scale;   // w8: (N, K/group) fp16
  const uint16_t* w16;     // fp16 weights (N, K) (when codes == nullptr)
  int group;
  uint16_t* y16;           // fp16 out (M, y_ld)
  int64_t y_ld;
  const uint16_t* resid;   // optional fp16 residual (M, resid_ld)
  int64_t resid_ld;
  int splits;              // K ranges (blockIdx.y); > 1 writes fp32 partials
  float* part;             // (splits, M, N) fp32 partials when splits > 1
  int row_out;             // fp16 rows written as 16-byte chunks (set by the host)
};

template <bool W8, int BM, int BN, int WM = 2>
__global__ __launch_bounds__(128 * WM) void gemm_kernel(const GemmArgs a) {
  using TL = Tile<BM, BN, WM, 2>;
  __shared__ __align__(16) uint16_t lds[TL::LDS_ELEMS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int64_t nbm = (a.M + BM - 1) / BM, nbn = (a.N + BN - 1) / BN;
  const int64_t tile = xcd_tile(blockIdx.x, nbm * nbn);
  const int64_t m0 = (tile % nbm) * BM, n0 = (tile / nbm) * BN;
  const int z = blockIdx.y;
  const int64_t klen = a.K / a.splits, kb = z * klen;  // this block's K range

  Sources<TL, W8> src;
#pragma unroll
  for (int i = 0; i < TL::A_CH; ++i) {
    int64_t m = m0 + TL::a_row(t, i);
    m = m < a.M ? m : a.M - 1;
    const int64_t row = a.x_rows ? (int64_t)a.x_rows[m] : m;
    src.a[i] = a.x + row * a.x_ld + kb + TL::a_col(t, i);
  }
  if constexpr (W8) {
    const int64_t ng = a.K / a.group;
#pragma unroll
    for (int i = 0; i < TL::B8_CH; ++i) {
      int64_t n = n0 + TL::b8_row(t, i);
      n = n < a.N ? n : a.N - 1;
      src.bc[i] = a.codes + n * a.K + kb + TL::b8_col(t, i);
      src.bs[i] = a.scale + n * ng + kb / a.group;
    }
  } else {
#pragma unroll
    for (int i = 0; i < TL::B16_CH; ++i) {
      int64_t n = n0 + TL::b16_row(t, i);
      n = n < a.N ? n : a.N - 1;
      src.bw[i] = a.w16 + n * a.K + kb + TL::b16_col(t, i);
    }
  }
  const int wm = wave >> 1, wn = wave & 1;  // WM x 2 waves
  int b_row0[TL::FN];
#pragma unroll
  for (int j = 0; j < TL::FN; ++j) b_row0[j] = wn * (BN / 2) + 32 * j;
  Acc<TL::FM, TL::FN> acc;
  block_mainloop2<TL, W8>(acc, src, klen, a.group, lds, wm * (BM / WM), b_row0);

  if (a.row_out) {  // block-uniform
    // fp16(acc) into the (then idle) stage buffers as a BM x BN row-major
    // tile, then each row segment goes out in 16-byte chunks with the
    // residual added per chunk: the same roundings as the per-element path.
    constexpr int OP = BN + 8, CPR = BN / 8, RPI = TL::NT / CPR;
    static_assert(BM * OP <= TL::LDS_ELEMS && TL::NT % CPR == 0, "output tile");
    __syncthreads();  // every wave has read its last stage from LDS
#pragma unroll
    for (int i = 0; i < TL::FM; ++i)
#pragma unroll
      for (int j = 0; j < TL::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          lds[(wm * (BM / WM) + 32 * i + acc_row(r, half)) * OP + wn * (BN / 2) + 32 * j + l32] =
              f2h(acc.v[i][j][r]);
    __syncthreads();
    const int c8 = (t % CPR) * 8;
    const int64_t n = n0 + c8;
    if (n >= a.N) return;  // N % 8 == 0: a chunk is wholly inside or outside
    const int rows = (int)(a.M - m0 < BM ? a.M - m0 : BM);
    for (int row = t / CPR; row < rows; row += RPI) {
      u32x4 v = *reinterpret_cast<const u32x4*>(lds + row * OP + c8);
      if (a.resid) {
        const u32x4 rv = *reinterpret_cast<const u32x4*>(a.resid + (m0 + row) * a.resid_ld + n);
        const uint32_t in[4] = {v.x, v.y, v.z, v.w}, ri[4] = {rv.x, rv.y, rv.z, rv.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint16_t lo = hadd_round(h2f((uint16_t)(in[q] & 0xFFFFu)), (uint16_t)(ri[q] & 0xFFFFu));
          const uint16_t hi = hadd_round(h2f((uint16_t)(in[q] >> 16)), (uint16_t)(ri[q] >> 16));
          o[q] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        v = (u32x4){o[0], o[1], o[2], o[3]};
      }
      *reinterpret_cast<u32x4*>(a.y16 + (m0 + row) * a.y_ld + n) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TL::FM; ++i)
#pragma unroll
    for (int j = 0; j < TL::FN; ++j) {
      const int64_t n = n0 + wn * (BN / 2) + 32 * j + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * (BM / WM) + 32 * i + acc_row(r, half);
        if (m >= a.M || n >= a.N) continue;
        if (a.part) {
          a.part[((int64_t)z * a.M + m) * a.N + n] = acc.v[i][j][r];
          continue;
        }
        uint16_t o = f2h(acc.v[i][j][r]);
        if (a.resid) o = hadd_round(h2f(o), a.resid[m * a.resid_ld + n]);
        a.y16[m * a.y_ld + n] = o;
      }
    }
}

// Split-K finish: y = fp16(sum over z of part[z]) in z order (+ residual).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int splits, int64_t M,
                                                           int64_t N, uint16_t* __restrict__ y, int64_t y_ld,
                                                           const uint16_t* __restrict__ resid, int64_t resid_ld) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx - m * N;
  float v = 0.0f;
  for (int z = 0; z < splits; ++z) v += part[z * M * N + idx];
  uint16_t o = f2h(v);
  if (resid) o = hadd_round(h2f(o), resid[m * resid_ld + n]);
  y[m * y_ld + n] = o;
}

template <bool W8>
int launch_tiles(const GemmArgs& a, hipStream_t st) {
  if (a.splits > 1) {  // small grids: 64 x 64 tiles, one K range per blockIdx.y, then the ordered sum
    const int64_t tiles = ((a.M + 63) / 64) * ((a.N + 63) / 64);
    hipLaunchKernelGGL((gemm_kernel<W8, 64, 64>), dim3((unsigned)tiles, (unsigned)a.splits), dim3(256), 0, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    if (!a.y16) return LEMOQ_OK;  // partials only: the consumer sums them
    const int64_t n = a.M * a.N;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a.part, a.splits,
                       a.M, a.N, a.y16, a.y_ld, a.resid, a.resid_ld);
    LEMOQ_CHECK_LAUNCH();
  }
  // Measured on the OLMoE linears (qkv, o_proj at 1 to 4096 rows): 256 x 128 tiles of 8
  // waves (each wave 64 x 64, the B tile shared by 4 row waves) are fastest while they give
  // at least 192 blocks; then 128 x 128 (8 waves of 32 x 64) from 256 blocks; below that, and
  // for fewer rows than a tile (padding rows cost matrix work), 64 x 64 tiles of 4 waves.
  const int64_t t256 = ((a.M + 255) / 256) * ((a.N + 127) / 128);
  const int64_t t128 = ((a.M + 127) / 128) * ((a.N + 127) / 128);
  if (a.M >= 256 && t256 >= 192) {
    hipLaunchKernelGGL((gemm_kernel<W8, 256, 128, 4>), dim3((unsigned)t256), dim3(512), 0, st, a);
  } else if (a.M >= 128 && t128 >= 256) {
    hipLaunchKernelGGL((gemm_kernel<W8, 128, 128, 4>), dim3((unsigned)t128), dim3(512), 0, st, a);
  } else {
    const int64_t small = ((a.M + 63) / 64) * ((a.N + 63) / 64);
    hipLaunchKernelGGL((gemm_kernel<W8, 64, 64>), dim3((unsigned)small), dim3(256), 0, st, a);
  }
  LEMOQ_CHECK_LAUNCH();
}

int launch_gemm(GemmArgs a, hipStream_t st) {
  // 16-byte row stores need 16-byte aligned rows of the output (and residual)
  a.row_out = a.splits == 1 && a.y16 && lemoq_aligned16(a.y16) && a.y_ld % 8 == 0 && a.N % 8 == 0 &&
              (!a.resid || (lemoq_aligned16(a.resid) && a.resid_ld % 8 == 0));
  return a.codes ? launch_tiles<true>(a, st) : launch_tiles<false>(a, st);
}

int check_gemm(const GemmArgs& a) {
  if (!a.x || (!a.codes && !a.w16) || (a.codes && !a.scale) || (!a.y16 && (a.splits == 1 || a.resid)))
    return LEMOQ_ERR_NULL;
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.M > (1LL << 24) || a.N > (1LL << 24)) return LEMOQ_ERR_SHAPE;
  if (((a.M + 63) / 64) * ((a.N + 63) / 64) > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  if (a.K % 64 != 0 || a.x_ld < a.K || a.x_ld % 8 != 0 || (a.y16 && a.y_ld < a.N)) return LEMOQ_ERR_SHAPE;
  if (a.codes && (a.group <= 0 || a.group % 64 != 0 || a.K % a.group != 0)) return LEMOQ_ERR_UNSUPPORTED;
  if (a.resid && a.resid_ld < a.N) return LEMOQ_ERR_SHAPE;
  if (a.splits < 1 || a.splits > 64 || a.K % (64LL * a.splits) != 0) return LEMOQ_ERR_SHAPE;
  if (a.splits > 1 && (!a.part || (a.codes && (a.K / a.splits) % a.group != 0) || a.M * a.N > (1LL << 31)))
    return a.part ? LEMOQ_ERR_SHAPE : LEMOQ_ERR_NULL;
  if (!lemoq_aligned16(a.x) || (a.codes && !lemoq_aligned16(a.codes)) || (a.w16 && !lemoq_aligned16(a.w16)))
    return LEMOQ_ERR_ALIGN;
  return LEMOQ_OK;
}

}  // namespace

extern "C" int lemoq_gemm_w8(const uint16_t* x, int64_t M, int64_t K, int64_t x_ld, const int32_t* x_rows,
                             const int8_t* codes, const uint16_t* scale, int64_t N, int64_t group,
                             uint16_t* y, int64_t y_ld, const uint16_t* residual, int64_t residual_ld,
                             void* stream) {
  GemmArgs a{};
  a.x = x; a.x_ld = x_ld; a.x_rows = x_rows; a.M = M; a.N = N; a.K = K;
  a.codes = codes; a.scale = scale; a.w16 = nullptr; a.group = (int)group;
  a.y16 = y; a.y_ld = y_ld;
  a.resid = residual; a.resid_ld = residual_ld;
  a.splits = 1; a.part = nullptr;
  if (!y || !codes) return LEMOQ_ERR_NULL;
  const int rc = check_gemm(a);
  if (rc != LEMOQ_OK) return rc;
  return launch_gemm(a, lemoq_stream(stream));
}

extern "C" int lemoq_gemm_f16(const uint16_t* x, int64_t M, int64_t K, int64_t x_ld, const uint16_t* w,
                              int64_t N, uint16_t* y, int64_t y_ld, void* stream) {
  GemmArgs a{};
  a.x = x; a.x_ld = x_ld; a.x_rows = nullptr; a.M = M; a.N = N; a.K = K;
  a.codes = nullptr; a.scale = nullptr; a.w16 = w; a.group = 0;
  a.y16 = y; a.y_ld = y_ld;
  a.resid = nullptr; a.resid_ld = 0;
  a.splits = 1; a.part = nullptr;
  if (!y || !w) return LEMOQ_ERR_NULL;
  const int rc = check_gemm(a);
  if (rc != LEMOQ_OK) return rc;
  return launch_gemm(a, lemoq_stream(stream));
}

// ---------------------------------------------------------------------------
// lemoq_gemm_f16_splitk_noalloc: the same launches with the split partials in
// a fixed device array instead of a caller workspace, so the call allocates
// nothing.  The array's host-side name is not a device address: its address
// on each device comes from hipGetSymbolAddress, taken once per device (with
// that device current) on the first call there, and only that pointer is
// handed to the kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[LEMOQ_SPLITK_SCRATCH_FLOATS];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch` (looked up once per device).
int scratch_ptr(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return LEMOQ_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return LEMOQ_ERR_NULL;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return LEMOQ_OK;
}

}  // namespace

extern "C" int lemoq_gemm_f16_splitk_noalloc(const uint16_t* x, int64_t M, int64_t K, int64_t x_ld,
                                             const uint16_t* w, int64_t N, uint16_t* y, int64_t y_ld,
                                             int64_t splits, void* stream) {
  GemmArgs a{};
  a.x = x; a.x_ld = x_ld; a.x_rows = nullptr; a.M = M; a.N = N; a.K = K;
  a.codes = nullptr; a.scale = nullptr; a.w16 = w; a.group = 0;
  a.y16 = y; a.y_ld = y_ld;
  a.resid = nullptr; a.resid_ld = 0;
  // y is required: the partials stay in the library's array, which the caller cannot read
  if (!y || !w) return LEMOQ_ERR_NULL;
  if (splits < 1 || splits > 64) return LEMOQ_ERR_SHAPE;
  if (M <= 0 || N <= 0 || M > (1LL << 24) || N > (1LL << 24)) return LEMOQ_ERR_SHAPE;
  if (splits > 1 && M * N > LEMOQ_SPLITK_SCRATCH_FLOATS / splits) return LEMOQ_ERR_CAPACITY;
  a.splits = (int)splits;
  a.part = nullptr;
  if (splits > 1) {
    const int rc = scratch_ptr(&a.part);
    if (rc != LEMOQ_OK) return rc;
  }
  const int rc = check_gemm(a);
  if (rc != LEMOQ_OK) return rc;
  return launch_gemm(a, lemoq_stream(stream));
}

extern "C" int lemoq_gemm_f16_splitk(const uint16_t* x, int64_t M, int64_t K, int64_t x_ld, const uint16_t* w,
                                     int64_t N, uint16_t* y, int64_t y_ld, int64_t splits, float* workspace,
                                     void* stream) {
  GemmArgs a{};
  a.x = x; a.x_ld = x_ld; a.x_rows = nullptr; a.M = M; a.N = N; a.K = K;
  a.codes = nullptr; a.scale = nullptr; a.w16 = w; a.group = 0;
  a.y16 = y; a.y_ld = y_ld;
  a.resid = nullptr; a.resid_ld = 0;
  if ((!y && splits == 1) || !w) return LEMOQ_ERR_NULL;
  if (splits < 1 || splits > 64) return LEMOQ_ERR_SHAPE;
  a.splits = (int)splits;
  // one split is lemoq_gemm_f16: the workspace is not used (a non-null part
  // would make the kernel write partials instead of y)
  a.part = splits > 1 ? workspace : nullptr;
  if (splits > 1 && !lemoq_aligned16(workspace)) return workspace ? LEMOQ_ERR_ALIGN : LEMOQ_ERR_NULL;
  const int rc = check_gemm(a);
  if (rc != LEMOQ_OK) return rc;
  return launch_gemm(a, lemoq_stream(stream));
}
