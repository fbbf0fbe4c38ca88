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
// Tiling: 4 waves per block as 2 x 2 wave tiles of 64 x 64 (the main loop of
// gemm_core.h), no LDS.
//
// Rows: X row m may be gathered (x_rows[m]); the output is fp16 rows with an
// optional fp16 residual added in one rounding (torch's fp16 add).  Rows and
// columns beyond M/N are clamped on load and not stored.
#include "gemm_core.h"

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
};

template <bool W8, int FM, int FN>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  constexpr int TM = 32 * FM, TN = 32 * FN;
  const int64_t m0 = ((int64_t)blockIdx.y * 2 + (wave >> 1)) * TM;
  const int64_t n0 = ((int64_t)blockIdx.x * 2 + (wave & 1)) * TN;
  if (m0 >= a.M || n0 >= a.N) return;  // wave-uniform: a whole wave tile outside the output

  const uint16_t* xr[FM];
#pragma unroll
  for (int f = 0; f < FM; ++f) {
    int64_t m = m0 + 32 * f + l32;
    m = m < a.M ? m : a.M - 1;
    const int64_t src = a.x_rows ? (int64_t)a.x_rows[m] : m;
    xr[f] = a.x + src * a.x_ld + 16 * half;
  }
  WRow wr[FN];
  const int64_t ng = W8 ? a.K / a.group : 1;
#pragma unroll
  for (int f = 0; f < FN; ++f) {
    int64_t n = n0 + 32 * f + l32;
    n = n < a.N ? n : a.N - 1;
    wr[f].codes = W8 ? a.codes + n * a.K + 16 * half : nullptr;
    wr[f].scale = W8 ? a.scale + n * ng : nullptr;
    wr[f].w16 = W8 ? nullptr : a.w16 + n * a.K + 16 * half;
  }
  Acc<FM, FN> acc;
  acc_zero(acc);
  mainloop<W8>(acc, xr, wr, a.K, a.group);

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t n = n0 + 32 * j + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + 32 * i + acc_row(r, half);
        if (m >= a.M || n >= a.N) continue;
        uint16_t o = f2h(acc.v[i][j][r]);
        if (a.resid) o = hadd_round(h2f(o), a.resid[m * a.resid_ld + n]);
        a.y16[m * a.y_ld + n] = o;
      }
    }
}

int launch_gemm(const GemmArgs& a, hipStream_t st) {
  constexpr int FM = 2, FN = 2;
  const dim3 grid((unsigned)((a.N + 2 * 32 * FN - 1) / (2 * 32 * FN)),
                  (unsigned)((a.M + 2 * 32 * FM - 1) / (2 * 32 * FM)));
  if (a.codes)
    hipLaunchKernelGGL((gemm_kernel<true, FM, FN>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_kernel<false, FM, FN>), grid, dim3(256), 0, st, a);
  LEMOQ_CHECK_LAUNCH();
}

int check_gemm(const GemmArgs& a) {
  if (!a.x || (!a.codes && !a.w16) || (a.codes && !a.scale) || !a.y16) return LEMOQ_ERR_NULL;
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.M > 65535LL * 128 || a.N > 65535LL * 128) return LEMOQ_ERR_SHAPE;
  if (a.K % 32 != 0 || a.x_ld < a.K || a.x_ld % 8 != 0 || a.y_ld < a.N) return LEMOQ_ERR_SHAPE;
  if (a.codes && (a.group <= 0 || a.group % 32 != 0 || a.K % a.group != 0)) return LEMOQ_ERR_UNSUPPORTED;
  if (a.resid && a.resid_ld < a.N) return LEMOQ_ERR_SHAPE;
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
  if (!y || !w) return LEMOQ_ERR_NULL;
  const int rc = check_gemm(a);
  if (rc != LEMOQ_OK) return rc;
  return launch_gemm(a, lemoq_stream(stream));
}
