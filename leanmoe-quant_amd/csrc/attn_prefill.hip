// Causal self-attention over the prompt (prefill) on the matrix cores.
//
// The reference prefills through HF's attention with the sdpa backend (the
// decode core replacement only takes q_len == 1; src/lemoq/kernels/
// attn_decode.py:836-1017): softmax(q k^T / sqrt(D) + causal mask) v over the
// fp16 q, k, v of the prompt, fp32 inside, fp16 out.  This kernel computes
// the same with an online softmax (flash-attention order), fp32 statistics
// and accumulators; P is rounded to fp16 for the P V product (as flash
// kernels do).
//
// Layout per wave: 32 queries; key tiles of 32.  S^T = K Q^T puts one query
// per lane column (accumulator register r of lane l holds key
// 8*(r/4) + 4*(l/32) + r%4, query l % 32), so the running max and sum of a
// query are a lane-local reduction plus one exchange with lane l ^ 32, and
// the probabilities are already the B operand of O^T = V^T P^T (with the key
// order of that register layout used for the k index of both operands).  The
// V tile is staged transposed in LDS (V^T rows of 32 keys); the K tile is
// staged row-major.  A block of NW waves (32*NW queries) shares the tiles;
// blocks are launched heaviest (latest queries) first.
#include "common.h"

namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int KT = 32;  // keys per tile

__device__ __forceinline__ h8v h8_of(const u32x4 v) { return __builtin_bit_cast(h8v, v); }

template <int D, int NW>
__global__ __launch_bounds__(64 * NW) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t q_ld, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int64_t kv_head_stride, int64_t T, float qk_scale,
    uint16_t* __restrict__ out, int64_t out_ld) {
  constexpr int QB = 32 * NW;
  constexpr int KP = D + 8;   // K tile row pitch (fp16): 16-byte pad
  constexpr int VP = KT + 4;  // V^T row pitch (fp16): 8-byte pad
  constexpr int DF = D / 32;  // output fragments (32 dims each)
  __shared__ __align__(16) uint16_t ks[KT * KP];
  __shared__ __align__(16) uint16_t vt[D * VP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int h = blockIdx.y;
  const int64_t nqb = (T + QB - 1) / QB;
  const int64_t q0 = (nqb - 1 - (int64_t)blockIdx.x) * QB;
  const int64_t qw = q0 + 32 * wave;
  const int64_t qi = qw + l32;
  const int64_t qc = qi < T ? qi : T - 1;

  // Q^T operand: lane half h holds dims 32j + 16h + [0, 16) of its query.
  h8v qf[DF][2];
  {
    const uint16_t* qp = q + qc * q_ld + (int64_t)h * D + 16 * half;
#pragma unroll
    for (int j = 0; j < DF; ++j) {
      qf[j][0] = h8_of(*reinterpret_cast<const u32x4*>(qp + 32 * j));
      qf[j][1] = h8_of(*reinterpret_cast<const u32x4*>(qp + 32 * j + 8));
    }
  }
  const uint16_t* kh = k + (int64_t)h * kv_head_stride;
  const uint16_t* vh = v + (int64_t)h * kv_head_stride;

  float m = -INFINITY, l = 0.0f;
  f32x16 o[DF];
#pragma unroll
  for (int f = 0; f < DF; ++f) o[f] = (f32x16){};

  const int64_t kend = T < q0 + QB ? T : q0 + QB;
  for (int64_t k0 = 0; k0 < kend; k0 += KT) {
    __syncthreads();  // the previous tile has been read
    for (int c = threadIdx.x; c < KT * D / 8; c += 64 * NW) {
      const int kr = c / (D / 8), c8 = c - kr * (D / 8);
      int64_t key = k0 + kr;
      key = key < T ? key : T - 1;
      const u32x4 kv = *reinterpret_cast<const u32x4*>(kh + key * D + c8 * 8);
      const u32x4 vv = *reinterpret_cast<const u32x4*>(vh + key * D + c8 * 8);
      *reinterpret_cast<u32x4*>(ks + kr * KP + c8 * 8) = kv;
      const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt[(c8 * 8 + 2 * e) * VP + kr] = (uint16_t)(w[e] & 0xFFFFu);
        vt[(c8 * 8 + 2 * e + 1) * VP + kr] = (uint16_t)(w[e] >> 16);
      }
    }
    __syncthreads();
    if (k0 > qw) continue;  // wave-uniform: every key of the tile is after every query of the wave

    // S^T (32 keys x 32 queries)
    f32x16 s = (f32x16){};
#pragma unroll
    for (int j = 0; j < DF; ++j) {
      const uint16_t* kp = ks + l32 * KP + 32 * j + 16 * half;
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of(*reinterpret_cast<const u32x4*>(kp)), qf[j][0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of(*reinterpret_cast<const u32x4*>(kp + 8)), qf[j][1], s, 0,
                                                 0, 0);
    }
    float x[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t key = k0 + 8 * (r / 4) + 4 * half + (r % 4);
      x[r] = (key <= qi && key < T) ? s[r] * qk_scale : -INFINITY;
      mx = fmaxf(mx, x[r]);
    }
    mx = fmaxf(mx, xor32_get(mx, lane));
    // key k0 <= qw <= qi is valid for every query, so mn is finite
    const float mn = fmaxf(m, mx);
    const float alpha = exp2f(m - mn);
    float ps = 0.0f;
    uint32_t pk[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p0 = exp2f(x[2 * i] - mn), p1 = exp2f(x[2 * i + 1] - mn);
      ps += p0 + p1;
      pk[i] = (uint32_t)f2h(p0) | ((uint32_t)f2h(p1) << 16);
    }
    l = l * alpha + ps;
    m = mn;
    const h8v pb0 = h8_of((u32x4){pk[0], pk[1], pk[2], pk[3]});
    const h8v pb1 = h8_of((u32x4){pk[4], pk[5], pk[6], pk[7]});
#pragma unroll
    for (int f = 0; f < DF; ++f) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[f][r] *= alpha;
      const uint16_t* vp = vt + (32 * f + l32) * VP + 4 * half;
      const uint2 a0 = *reinterpret_cast<const uint2*>(vp);
      const uint2 a1 = *reinterpret_cast<const uint2*>(vp + 8);
      const uint2 b0 = *reinterpret_cast<const uint2*>(vp + 16);
      const uint2 b1 = *reinterpret_cast<const uint2*>(vp + 24);
      o[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of((u32x4){a0.x, a0.y, a1.x, a1.y}), pb0, o[f], 0, 0, 0);
      o[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of((u32x4){b0.x, b0.y, b1.x, b1.y}), pb1, o[f], 0, 0, 0);
    }
  }

  const float lt = l + xor32_get(l, lane);
  const float inv = 1.0f / lt;
  if (qi >= T) return;
  uint16_t* op = out + qi * out_ld + (int64_t)h * D + 4 * half;
#pragma unroll
  for (int f = 0; f < DF; ++f)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t lo = (uint32_t)f2h(o[f][4 * b] * inv) | ((uint32_t)f2h(o[f][4 * b + 1] * inv) << 16);
      const uint32_t hi = (uint32_t)f2h(o[f][4 * b + 2] * inv) | ((uint32_t)f2h(o[f][4 * b + 3] * inv) << 16);
      *reinterpret_cast<uint2*>(op + 32 * f + 8 * b) = make_uint2(lo, hi);
    }
}

}  // namespace

extern "C" int lemoq_attn_prefill_f16(const uint16_t* q, int64_t q_ld, const uint16_t* k, const uint16_t* v,
                                      int64_t kv_head_stride, int64_t T, int64_t heads, int64_t head_dim,
                                      float qk_scale, uint16_t* out, int64_t out_ld, void* stream) {
  if (!q || !k || !v || !out) return LEMOQ_ERR_NULL;
  if (T <= 0 || heads <= 0 || heads > 65535) return LEMOQ_ERR_SHAPE;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (q_ld < heads * head_dim || out_ld < heads * head_dim || q_ld % 8 != 0 || out_ld % 4 != 0 ||
      kv_head_stride < T * head_dim || kv_head_stride % 8 != 0)
    return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(q) || !lemoq_aligned16(k) || !lemoq_aligned16(v) ||
      (reinterpret_cast<uintptr_t>(out) & 7u) != 0)
    return LEMOQ_ERR_ALIGN;
  constexpr int NW = 2;
  const int64_t nqb = (T + 32 * NW - 1) / (32 * NW);
  if (nqb > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  const dim3 grid((unsigned)nqb, (unsigned)heads);
  hipStream_t st = lemoq_stream(stream);
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL((attn_prefill_kernel<64, NW>), grid, dim3(64 * NW), 0, st, q, q_ld, k, v,
                         kv_head_stride, T, qk_scale, out, out_ld);
      break;
    case 128:
      hipLaunchKernelGGL((attn_prefill_kernel<128, NW>), grid, dim3(64 * NW), 0, st, q, q_ld, k, v,
                         kv_head_stride, T, qk_scale, out, out_ld);
      break;
    default:
      hipLaunchKernelGGL((attn_prefill_kernel<256, NW>), grid, dim3(64 * NW), 0, st, q, q_ld, k, v,
                         kv_head_stride, T, qk_scale, out, out_ld);
      break;
  }
  LEMOQ_CHECK_LAUNCH();
}
