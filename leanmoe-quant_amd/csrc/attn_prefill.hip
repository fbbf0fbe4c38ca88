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
// Layout per wave: 32 queries.  S^T = K Q^T puts one query per lane column
// (accumulator register r of lane l holds key 8*(r/4) + 4*(l/32) + r%4 of the
// 32-key fragment, query l % 32), so the running max and sum of a query are a
// lane-local reduction plus one exchange with lane l ^ 32, and the
// probabilities are already the B operand of O^T = V^T P^T (with the key
// order of that register layout used for the k index of both operands).
//
// A block of NW waves shares key tiles of KT = 8192 / D keys staged in LDS:
// K row-major, V transposed (V^T rows of KT keys).  Each wave owns 32
// queries; with a key split KS = 2, two waves own the same 32 queries and
// take the two halves of every tile, and their online-softmax states are
// merged through LDS at the end (more blocks for short prompts).  The tile
// after the current one is loaded into registers before the current one is
// used (V as 4-key x 8-dim sub-blocks, transposed in registers so the LDS
// writes are 8 bytes wide) and written to the other half of a double buffer;
// one barrier per tile.  Blocks are launched heaviest (latest queries) first,
// or paired with complementary work on one CU (attn_block_of).
#include "common.h"

namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ h8v h8_of(const u32x4 v) { return __builtin_bit_cast(h8v, v); }

// 2^x by v_exp_f32 alone, for the softmax numerators and the running-max
// rescale.  Results below 2^-126 flush to 0 where exp2f returns denormals; p
// is rounded to fp16 (smallest subnormal 2^-24) before P.V and every running
// sum it enters is >= 1, so no output changes.  exp2f's denormal path costs
// four more instructions per score.
__device__ __forceinline__ float exp2_flush(float x) { return __builtin_amdgcn_exp2f(x); }

template <int D, int NW, int KS = 1>
struct AttnGeom {
  static constexpr int THREADS = 64 * NW;
  static constexpr int QG = NW / KS;               // query fragments per block
  static constexpr int QB = 32 * QG;               // queries per block
  static constexpr int KT = 8192 / D;              // keys per tile
  static constexpr int NS = KT / 32;               // S fragments per tile
  static constexpr int NSW = NS / KS;              // S fragments per wave per tile
  static_assert(NS % KS == 0 && NW % KS == 0, "key split");
  static constexpr int DF = D / 32;                // output fragments
  static constexpr int KP = D + 8;                 // K tile row pitch (fp16)
  static constexpr int VP = KT + 8;                // V^T row pitch (fp16)
  static constexpr int K_CH = KT * D / 8 / THREADS;        // 16-byte K chunks per thread
  static constexpr int V_CH = (KT / 4) * (D / 8) / THREADS;  // 4 x 8 V sub-blocks per thread
  static constexpr int HALF = KT * KP + D * VP;    // fp16 per LDS buffer
  // V^T row r keeps its 16-byte key chunk c at chunk c ^ vswz(r): the stores
  // (8 bytes to rows 8 dq + 2 w) then spread over all banks instead of two.
  static constexpr int VCH = KT / 8;               // 16-byte key chunks per V^T row
  __device__ static int vswz(int r) { return (r >> 4) & (VCH - 1); }
  static_assert(K_CH >= 1 && V_CH >= 1, "tile split");
};

template <class G>
struct AttnStage {
  u32x4 k[G::K_CH];
  u32x4 v[G::V_CH][4];
};

template <int D, class G>
__device__ __forceinline__ void attn_load(AttnStage<G>& st, const uint16_t* __restrict__ kh,
                                          const uint16_t* __restrict__ vh, int64_t k0, int64_t T, int t) {
#pragma unroll
  for (int i = 0; i < G::K_CH; ++i) {
    const int c = t + G::THREADS * i;
    int64_t key = k0 + c / (D / 8);
    key = key < T ? key : T - 1;
    st.k[i] = *reinterpret_cast<const u32x4*>(kh + key * D + 8 * (c % (D / 8)));
  }
#pragma unroll
  for (int i = 0; i < G::V_CH; ++i) {
    const int c = t + G::THREADS * i;
    const int kq = c / (D / 8), dq = c % (D / 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int64_t key = k0 + 4 * kq + j;
      key = key < T ? key : T - 1;
      st.v[i][j] = *reinterpret_cast<const u32x4*>(vh + key * D + 8 * dq);
    }
  }
}

template <int D, class G>
__device__ __forceinline__ void attn_store(const AttnStage<G>& st, uint16_t* buf, int t) {
  uint16_t* ks = buf;
  uint16_t* vt = buf + G::KT * G::KP;
#pragma unroll
  for (int i = 0; i < G::K_CH; ++i) {
    const int c = t + G::THREADS * i;
    *reinterpret_cast<u32x4*>(ks + (c / (D / 8)) * G::KP + 8 * (c % (D / 8))) = st.k[i];
  }
#pragma unroll
  for (int i = 0; i < G::V_CH; ++i) {
    const int c = t + G::THREADS * i;
    const int kq = c / (D / 8), dq = c % (D / 8);
    const uint32_t v0[4] = {st.v[i][0].x, st.v[i][0].y, st.v[i][0].z, st.v[i][0].w};
    const uint32_t v1[4] = {st.v[i][1].x, st.v[i][1].y, st.v[i][1].z, st.v[i][1].w};
    const uint32_t v2[4] = {st.v[i][2].x, st.v[i][2].y, st.v[i][2].z, st.v[i][2].w};
    const uint32_t v3[4] = {st.v[i][3].x, st.v[i][3].y, st.v[i][3].z, st.v[i][3].w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      // dims 2w and 2w+1 of keys 4kq .. 4kq+3
      const uint2 lo = make_uint2(__builtin_amdgcn_perm(v1[w], v0[w], 0x05040100u),
                                  __builtin_amdgcn_perm(v3[w], v2[w], 0x05040100u));
      const uint2 hi = make_uint2(__builtin_amdgcn_perm(v1[w], v0[w], 0x07060302u),
                                  __builtin_amdgcn_perm(v3[w], v2[w], 0x07060302u));
      const int r0 = 8 * dq + 2 * w, r1 = r0 + 1;
      *reinterpret_cast<uint2*>(vt + r0 * G::VP + 8 * ((kq >> 1) ^ G::vswz(r0)) + 4 * (kq & 1)) = lo;
      *reinterpret_cast<uint2*>(vt + r1 * G::VP + 8 * ((kq >> 1) ^ G::vswz(r1)) + 4 * (kq & 1)) = hi;
    }
  }
}

// Query blocks and heads over the grid.  Two-dimensional: blockIdx.x is the
// query block's rank (0 = the latest prompt rows, the most keys), blockIdx.y
// the head.  PAIRED (an even number of heads): a 1-D grid whose first half
// takes heads 0 .. heads/2 - 1 latest-first and whose second half takes the
// other heads earliest-first, so blocks b and b + grid/2, which the dispatcher
// places on the same compute unit when the whole grid is resident at two
// blocks per CU, carry complementary numbers of key tiles.
template <bool PAIRED>
__device__ __forceinline__ void attn_block_of(int64_t nqb, int heads, int& h, int64_t& rank) {
  if constexpr (PAIRED) {
    const int64_t L = blockIdx.x, half_grid = nqb * (heads / 2);
    if (L < half_grid) {
      h = (int)(L / nqb);
      rank = L % nqb;
    } else {
      h = heads / 2 + (int)((L - half_grid) / nqb);
      rank = nqb - 1 - (L - half_grid) % nqb;
    }
  } else {
    h = blockIdx.y;
    rank = blockIdx.x;
  }
}

template <int D, int NW, int KS, bool PAIRED>
__device__ __forceinline__ void attn_prefill_body(
    const uint16_t* __restrict__ q, int64_t q_ld, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int64_t kv_head_stride, int64_t T, float qk_scale,
    uint16_t* __restrict__ out, int64_t out_ld, int heads) {
  using G = AttnGeom<D, NW, KS>;
  __shared__ __align__(16) uint16_t lds[2 * G::HALF];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int qfrag = wave % G::QG, kpart = wave / G::QG;  // kpart: which NSW-fragment slice of each tile
  const int64_t nqb = (T + G::QB - 1) / G::QB;
  int h;
  int64_t rank;
  attn_block_of<PAIRED>(nqb, heads, h, rank);
  const int64_t q0 = (nqb - 1 - rank) * G::QB;
  const int64_t qw = q0 + 32 * qfrag;
  const int64_t qi = qw + l32;
  const int64_t qc = qi < T ? qi : T - 1;

  // Q^T operand: lane half h holds dims 32j + 16h + [0, 16) of its query.
  h8v qf[G::DF][2];
  {
    const uint16_t* qp = q + qc * q_ld + (int64_t)h * D + 16 * half;
#pragma unroll
    for (int j = 0; j < G::DF; ++j) {
      qf[j][0] = h8_of(*reinterpret_cast<const u32x4*>(qp + 32 * j));
      qf[j][1] = h8_of(*reinterpret_cast<const u32x4*>(qp + 32 * j + 8));
    }
  }
  const uint16_t* kh = k + (int64_t)h * kv_head_stride;
  const uint16_t* vh = v + (int64_t)h * kv_head_stride;

  float m = -INFINITY, l = 0.0f;
  f32x16 o[G::DF];
#pragma unroll
  for (int f = 0; f < G::DF; ++f) o[f] = (f32x16){};

  const int64_t kend = T < q0 + G::QB ? T : q0 + G::QB;
  const int64_t ntile = (kend + G::KT - 1) / G::KT;
  AttnStage<G> st;
  attn_load<D, G>(st, kh, vh, 0, T, t);
  attn_store<D, G>(st, lds, t);
  __syncthreads();
  for (int64_t it = 0; it < ntile; ++it) {
    const int64_t k0 = it * G::KT;
    const int64_t kn = (it + 1 < ntile ? it + 1 : it) * G::KT;  // clamped prefetch
    attn_load<D, G>(st, kh, vh, kn, T, t);
    const uint16_t* ks = lds + (it & 1) * G::HALF;
    const uint16_t* vt = ks + G::KT * G::KP;
    const int64_t kw = k0 + 32 * G::NSW * kpart;  // first key of this wave's slice of the tile
    if (kw <= qw) {  // wave-uniform: the slice holds a key at or before every query of the wave
      f32x16 s[G::NSW];
#pragma unroll
      for (int sf = 0; sf < G::NSW; ++sf) s[sf] = (f32x16){};
      // K fragments of 32-dim chunk j + 1 are read from LDS while chunk j's
      // matrix ops run (AHEAD; read where they are used, each op waited for
      // its own read: 150 -> 131 us per layer at T 4096 with unsplit keys, no
      // gain with the key split); the NSW accumulation chains are interleaved
      // (independent neighbours).
      constexpr int AHEAD = KS == 1 ? 1 : 0;
      u32x4 kf[G::DF][2][G::NSW];
      auto kread = [&](int j) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int sf = 0; sf < G::NSW; ++sf)
            kf[j][hh][sf] = *reinterpret_cast<const u32x4*>(
                ks + (32 * (G::NSW * kpart + sf) + l32) * G::KP + 32 * j + 16 * half + 8 * hh);
      };
      if (AHEAD) kread(0);
#pragma unroll
      for (int j = 0; j < G::DF; ++j) {
        if (!AHEAD) kread(j);
        else if (j + 1 < G::DF) kread(j + 1);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int sf = 0; sf < G::NSW; ++sf)
            s[sf] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of(kf[j][hh][sf]), qf[j][hh], s[sf], 0, 0, 0);
      }
      float mx = -INFINITY;
      // Masks are needed only where the slice reaches past the wave's first
      // query or past the prompt (wave-uniform test); there the key offset
      // from this lane's query fits 32 bits.
      const int64_t kend_w = kw + 32 * G::NSW;
      if (kend_w - 1 <= qw && kend_w <= T) {
#pragma unroll
        for (int sf = 0; sf < G::NSW; ++sf)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s[sf][r] *= qk_scale;
            mx = fmaxf(mx, s[sf][r]);
          }
      } else {
        const int lim = (int)((T < qi + 1 ? T : qi + 1) - kw);  // keys kw + j with j < lim are valid
#pragma unroll
        for (int sf = 0; sf < G::NSW; ++sf)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int j = 32 * sf + 8 * (r / 4) + 4 * half + (r % 4);
            s[sf][r] = j < lim ? s[sf][r] * qk_scale : -INFINITY;
            mx = fmaxf(mx, s[sf][r]);
          }
      }
      mx = fmaxf(mx, xor32_get(mx, lane));
      // key kw <= qw <= qi is valid for every query of a wave with stored outputs
      // (qw < T), so mn is finite there; waves wholly past the prompt store nothing
      const float mn = fmaxf(m, mx);
      const float alpha = exp2_flush(m - mn);
      float ps = 0.0f;
      h8v pb[2 * G::NSW];
#pragma unroll
      for (int sf = 0; sf < G::NSW; ++sf) {
        uint32_t pk[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float p0 = exp2_flush(s[sf][2 * i] - mn), p1 = exp2_flush(s[sf][2 * i + 1] - mn);
          ps += p0 + p1;
          const f16x2 hp = {(f16)p0, (f16)p1};  // one v_cvt_pk_f16_f32 (round to nearest even)
          pk[i] = __builtin_bit_cast(uint32_t, hp);
        }
        pb[2 * sf] = h8_of((u32x4){pk[0], pk[1], pk[2], pk[3]});
        pb[2 * sf + 1] = h8_of((u32x4){pk[4], pk[5], pk[6], pk[7]});
      }
      l = l * alpha + ps;
      m = mn;
      // rescale only when some query's running max moved (wave-uniform test)
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int f = 0; f < G::DF; ++f)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[f][r] *= alpha;
      }
      // V^T fragments of 16-key step qq + 1 read during step qq's matrix ops (AHEAD)
      u32x4 vf[2 * G::NSW][G::DF];
      auto vread = [&](int qq) {
        const int kb = 32 * (G::NSW * kpart + qq / 2) + 16 * (qq % 2);
#pragma unroll
        for (int f = 0; f < G::DF; ++f) {
          const int vr = 32 * f + l32, sw = G::vswz(vr);  // keys kb + 4 half and kb + 8 + 4 half
          const uint16_t* vp = vt + vr * G::VP + 4 * half;
          const uint2 a0 = *reinterpret_cast<const uint2*>(vp + 8 * ((kb >> 3) ^ sw));
          const uint2 a1 = *reinterpret_cast<const uint2*>(vp + 8 * (((kb >> 3) + 1) ^ sw));
          vf[qq][f] = (u32x4){a0.x, a0.y, a1.x, a1.y};
        }
      };
      if (AHEAD) vread(0);
#pragma unroll
      for (int qq = 0; qq < 2 * G::NSW; ++qq) {
        if (!AHEAD) vread(qq);
        else if (qq + 1 < 2 * G::NSW) vread(qq + 1);
#pragma unroll
        for (int f = 0; f < G::DF; ++f)
          o[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of(vf[qq][f]), pb[qq], o[f], 0, 0, 0);
      }
    }
    attn_store<D, G>(st, lds + ((it + 1) & 1) * G::HALF, t);
    __syncthreads();
  }

  if constexpr (KS == 2) {
    // Merge the two key slices of each query fragment (the loop ended on a
    // barrier, so the tile buffers are free): slice 1 publishes m, its lane's
    // partial l and o, transposed so consecutive lanes hit consecutive banks;
    // slice 0 combines in a fixed order.
    constexpr int NV = 16 * G::DF + 2;
    float* mrg = reinterpret_cast<float*>(lds) + qfrag * NV * 64;
    if (kpart == 1) {
      mrg[lane] = m;
      mrg[64 + lane] = l;
#pragma unroll
      for (int f = 0; f < G::DF; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) mrg[(2 + 16 * f + r) * 64 + lane] = o[f][r];
    }
    __syncthreads();
    if (kpart == 1) return;
    const float mb = mrg[lane], lb = mrg[64 + lane];
    const float mm = fmaxf(m, mb);  // m is finite: slice 0 always holds key 0 for this fragment
    const float fa = exp2f(m - mm), fb = exp2f(mb - mm);
    l = l * fa + lb * fb;
#pragma unroll
    for (int f = 0; f < G::DF; ++f)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[f][r] = o[f][r] * fa + mrg[(2 + 16 * f + r) * 64 + lane] * fb;
  }
  const float lt = l + xor32_get(l, lane);
  const float inv = 1.0f / lt;
  if (qi >= T) return;
  uint16_t* op = out + qi * out_ld + (int64_t)h * D + 4 * half;
#pragma unroll
  for (int f = 0; f < G::DF; ++f)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t lo = (uint32_t)f2h(o[f][4 * b] * inv) | ((uint32_t)f2h(o[f][4 * b + 1] * inv) << 16);
      const uint32_t hi = (uint32_t)f2h(o[f][4 * b + 2] * inv) | ((uint32_t)f2h(o[f][4 * b + 3] * inv) << 16);
      *reinterpret_cast<uint2*>(op + 32 * f + 8 * b) = make_uint2(lo, hi);
    }
}

// Two waves per SIMD need at most 256 registers a lane: met without spills
// for head_dim 128 with 4-wave blocks (two blocks fit the LDS of a CU).
template <int D, int NW, int KS, bool PAIRED>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void attn_prefill_kernel_occ2(
    const uint16_t* __restrict__ q, int64_t q_ld, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int64_t kv_head_stride, int64_t T, float qk_scale,
    uint16_t* __restrict__ out, int64_t out_ld, int heads) {
  attn_prefill_body<D, NW, KS, PAIRED>(q, q_ld, k, v, kv_head_stride, T, qk_scale, out, out_ld, heads);
}

template <int D, int NW, int KS, bool PAIRED>
__global__ __launch_bounds__(64 * NW) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t q_ld, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int64_t kv_head_stride, int64_t T, float qk_scale,
    uint16_t* __restrict__ out, int64_t out_ld, int heads) {
  attn_prefill_body<D, NW, KS, PAIRED>(q, q_ld, k, v, kv_head_stride, T, qk_scale, out, out_ld, heads);
}

template <int D, int NW, int KS, bool PAIRED>
void launch_attn_grid(const uint16_t* q, int64_t q_ld, const uint16_t* k, const uint16_t* v,
                      int64_t kv_head_stride, int64_t T, int64_t heads, float qk_scale, uint16_t* out,
                      int64_t out_ld, hipStream_t st) {
  constexpr int QB = 32 * NW / KS;
  const int64_t nqb = (T + QB - 1) / QB;
  const dim3 grid = PAIRED ? dim3((unsigned)(nqb * heads)) : dim3((unsigned)nqb, (unsigned)heads);
  if constexpr (D == 128 && NW == 4)
    hipLaunchKernelGGL((attn_prefill_kernel_occ2<D, NW, KS, PAIRED>), grid, dim3(64 * NW), 0, st, q, q_ld, k, v,
                       kv_head_stride, T, qk_scale, out, out_ld, (int)heads);
  else
    hipLaunchKernelGGL((attn_prefill_kernel<D, NW, KS, PAIRED>), grid, dim3(64 * NW), 0, st, q, q_ld, k, v,
                       kv_head_stride, T, qk_scale, out, out_ld, (int)heads);
}

// 128-query blocks of an even number of heads run the paired grid: at ctx
// 4096 (512 blocks, the whole grid resident) 186 -> 157 us, at ctx 8192
// 648 -> 593 us, bit-identical.
template <int D, int NW, int KS>
void launch_attn(const uint16_t* q, int64_t q_ld, const uint16_t* k, const uint16_t* v, int64_t kv_head_stride,
                 int64_t T, int64_t heads, float qk_scale, uint16_t* out, int64_t out_ld, hipStream_t st) {
  constexpr int QB = 32 * NW / KS;
  const int64_t nqb = (T + QB - 1) / QB;
  if (KS == 1 && heads % 2 == 0 && nqb * heads <= 0x7fffffffLL)
    launch_attn_grid<D, NW, KS, true>(q, q_ld, k, v, kv_head_stride, T, heads, qk_scale, out, out_ld, st);
  else
    launch_attn_grid<D, NW, KS, false>(q, q_ld, k, v, kv_head_stride, T, heads, qk_scale, out, out_ld, st);
}

template <int D>
void launch_attn_d(const uint16_t* q, int64_t q_ld, const uint16_t* k, const uint16_t* v, int64_t kv_head_stride,
                   int64_t T, int64_t heads, float qk_scale, uint16_t* out, int64_t out_ld, hipStream_t st) {
  // 128 queries per 4-wave block once that gives two blocks per compute unit;
  // below that, 64 queries per block with each tile's keys split between
  // wave pairs (twice the blocks, half the keys per wave).
  if constexpr (D > 128) {  // one 32-key fragment per tile: nothing to split
    launch_attn<D, 4, 1>(q, q_ld, k, v, kv_head_stride, T, heads, qk_scale, out, out_ld, st);
  } else {
    if (((T + 127) / 128) * heads >= 512)
      launch_attn<D, 4, 1>(q, q_ld, k, v, kv_head_stride, T, heads, qk_scale, out, out_ld, st);
    else
      launch_attn<D, 4, 2>(q, q_ld, k, v, kv_head_stride, T, heads, qk_scale, out, out_ld, st);
  }
}

}  // namespace

extern "C" int lemoq_attn_prefill_f16(const uint16_t* q, int64_t q_ld, const uint16_t* k, const uint16_t* v,
                                      int64_t kv_head_stride, int64_t T, int64_t heads, int64_t head_dim,
                                      float qk_scale, uint16_t* out, int64_t out_ld, void* stream) {
  if (!q || !k || !v || !out) return LEMOQ_ERR_NULL;
  if (T <= 0 || T > (1LL << 30) || heads <= 0 || heads > 65535) return LEMOQ_ERR_SHAPE;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return LEMOQ_ERR_UNSUPPORTED;
  if (q_ld < heads * head_dim || out_ld < heads * head_dim || q_ld % 8 != 0 || out_ld % 4 != 0 ||
      kv_head_stride < T * head_dim || kv_head_stride % 8 != 0)
    return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(q) || !lemoq_aligned16(k) || !lemoq_aligned16(v) ||
      (reinterpret_cast<uintptr_t>(out) & 7u) != 0)
    return LEMOQ_ERR_ALIGN;
  hipStream_t st = lemoq_stream(stream);
  switch (head_dim) {
    case 64: launch_attn_d<64>(q, q_ld, k, v, kv_head_stride, T, heads, qk_scale, out, out_ld, st); break;
    case 128: launch_attn_d<128>(q, q_ld, k, v, kv_head_stride, T, heads, qk_scale, out, out_ld, st); break;
    default: launch_attn_d<256>(q, q_ld, k, v, kv_head_stride, T, heads, qk_scale, out, out_ld, st); break;
  }
  LEMOQ_CHECK_LAUNCH();
}
