// Device parts of the attention-output half of a decode layer (merge + o_proj
// per head group, residual + post-attention norm + router), launched by
// oproj_router.hip.
//
//   lemoq_attn_merge_o_proj_w8   the LSE merge of the split-KV partials fused
//                                into the w8 o_proj GEMV, split over groups of
//                                four heads (512 input features).  A block
//                                merges only its own four heads (one wave per
//                                head, the arithmetic of lemoq_attn_merge, so
//                                the fp16 attention output is bit-identical),
//                                then dots its 32 output rows with them and
//                                writes fp32 partial sums, one row of partials
//                                per head group.  lemoq_attn_merge_o_proj_w4 is
//                                the same on 4-bit codes (the w4a16 cell).
//   lemoq_router_logits_resid    o = fp16(sum of the partials in group order),
//                                h' = fp16(o + h) (the residual add after
//                                o_proj), xn = RMSNorm(h') (post-attention
//                                norm) and the router logits fp16(xn . W[e]).
//
// Merging in every o_proj block over all heads costs a 133 KB read per block
// (measured slower than the separate merge launch); the head-group split
// reads 33 KB of partials per o_proj block and 32 KB per router block.
//
// The roundings are those of the three separate launches: fp16 attention
// output, fp16 o_proj output, fp16 residual add (torch's), HF RMSNorm, fp16
// router logits with fp32 accumulation.  Only the fp32 summation order of the
// o_proj dot differs (per head group, then across groups).
#pragma once

#include "attn_common.h"
#include "qformat.h"

namespace lemoq_oproj {

constexpr int MO_D = 128;                  // head_dim of this path
constexpr int MO_HEADS = 4;                // heads per block column
constexpr int MO_COLS = MO_D * MO_HEADS;   // input features per block column
constexpr int MO_ROWS_WAVE = 8;            // 4 loads x 2 rows per wave
constexpr int MO_ROWS = 4 * MO_ROWS_WAVE;  // output rows per block

struct MergeOprojArgs {
  const float* m;    // (heads, NS) running max per split (log2 domain)
  const float* l;    // (heads, NS) running sum per split
  const float* acc;  // (heads, NS, 128) unnormalised outputs per split
  int NS;
  const int8_t* codes;    // (N, HD) int8, or (N, HD / 2) packed 4-bit codes
  const uint16_t* scale;  // (N, HD / group)
  int64_t N;
  int HD;
  int group;
  float* part;  // (HD / 512, N)
};

// Block (x, g): rows 32x .. 32x + 31 over input features [512 g, 512 g + 512).
// Wave w merges head 4g + w (lane holds dims lane and lane + 64) into LDS,
// then owns rows 32x + 8w .. + 7: lane l reads the 16 codes at feature
// 512 g + 16 (l % 32) of row 2i + l / 32 for i = 0..3 (a row slice is 512
// bytes, two rows per wave load).  Every load is issued at entry: the four
// weight slices and their scales first, then the merge inputs.
//
// Blocks are dispatched round-robin over the 8 XCDs (each with its own L2).
// With G = heads / 4 groups and R = N / 32 row blocks, linear block b goes to
// XCD b % 8; when G divides 8 and R * G is a multiple of 8, the blocks of XCD
// c all take head group c % G, so each L2 fetches one group's 33 KB of split
// partials instead of every group's.
// The weight slices of one o_proj tile (block (rb, g)), issued first.
struct OprojTile {
  u32x4 c[4];
  uint16_t s[4];
  int64_t row0;
  int g;
};

__device__ __forceinline__ void oproj_issue(const MergeOprojArgs& a, int g, int rb, OprojTile& t) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  t.g = g;
  t.row0 = (int64_t)rb * MO_ROWS + wave * MO_ROWS_WAVE;
  const int k0 = g * MO_COLS + 16 * l32;
  const int ngroups = a.HD / a.group;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = t.row0 + 2 * i + half;
    t.c[i] = load_stream16(a.codes + row * a.HD + k0);
    t.s[i] = a.scale[row * ngroups + k0 / a.group];
  }
}

// 4-bit codes (two per byte): a row slice of 512 features is 256 bytes, so one
// wave load covers 4 rows: lane l reads the 32 codes at feature 512 g +
// 32 (l % 16) of row 4i + l / 16 for i = 0, 1.
struct OprojTileQ4 {
  u32x4 c[2];
  uint16_t s[2];
  int64_t row0;
  int g;
};

__device__ __forceinline__ void oproj_issue_q4(const MergeOprojArgs& a, int g, int rb, OprojTileQ4& t) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  t.g = g;
  t.row0 = (int64_t)rb * MO_ROWS + wave * MO_ROWS_WAVE;
  const int k0 = g * MO_COLS + 32 * l16;
  const int row_bytes = a.HD / 2, ngroups = a.HD / a.group;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t row = t.row0 + 4 * i + q;
    t.c[i] = load_stream16(a.codes + row * row_bytes + k0 / 2);
    t.s[i] = a.scale[row * ngroups + k0 / a.group];
  }
}

// The LSE merge of the block's 4 heads into LDS (xs: 512 fp16), one wave per
// head (lane holds dims lane and lane + 64).
template <int NSMAX>
__device__ __forceinline__ void oproj_merge(const MergeOprojArgs& a, int g, uint16_t* xs) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int NS = a.NS;
  const int64_t hh = (int64_t)g * MO_HEADS + wave;
  const int jl = lane < NS ? lane : NS - 1;
  const float mraw = a.m[hh * NS + jl];
  const float lraw = a.l[hh * NS + jl];
  const float* ah = a.acc + hh * NS * MO_D + lane;
  float a0[NSMAX], a1[NSMAX];
#pragma unroll
  for (int j = 0; j < NSMAX; ++j) {
    const int64_t o = (int64_t)(j < NS ? j : NS - 1) * MO_D;
    a0[j] = ah[o];
    a1[j] = ah[o + 64];
  }
  LEMOQ_LOADS_ISSUED();

  float den;
  const float wj = lemoq_attn::lse_weight(mraw, lraw, lane, NS, den);
  xs[wave * MO_D + lane] = lemoq_attn::lse_out<NSMAX>(a0, wj, den);
  xs[wave * MO_D + 64 + lane] = lemoq_attn::lse_out<NSMAX>(a1, wj, den);
  __syncthreads();
}

// Merge, then the 4-bit tile's partial sums (rows 4i + r in lanes 16r .. 16r + 15).
template <int NSMAX>
__device__ __forceinline__ void oproj_finish_q4(const MergeOprojArgs& a, const OprojTileQ4& t, uint16_t* xs) {
  oproj_merge<NSMAX>(a, t.g, xs);
  const int lane = threadIdx.x & 63, l16 = lane & 15;
  XChunk x0, x1;
  load_xchunk(xs + 32 * l16, x0);
  load_xchunk(xs + 32 * l16 + 16, x1);
  float tot[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float v = h2f(t.s[i]) * lemoq_qf::dot32_i4<true>(t.c[i], x0, x1, 0.0f);
    v = lemoq_attn::group_sum_lanes<16>(v, lane);  // every lane holds its 16-lane row's total
#pragma unroll
    for (int r = 0; r < 4; ++r) tot[i][r] = lane_f(v, 16 * r);
  }
  float out = 0.0f;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (lane == 4 * i + r) out = tot[i][r];
  if (lane < MO_ROWS_WAVE) a.part[(int64_t)t.g * a.N + t.row0 + lane] = out;
}

// Merge the tile's 4 heads into LDS (xs: 512 fp16) and write its partial
// sums.
template <int NSMAX>
__device__ __forceinline__ void oproj_finish(const MergeOprojArgs& a, const OprojTile& t, uint16_t* xs) {
  oproj_merge<NSMAX>(a, t.g, xs);
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31;

  XChunk xc;
  load_xchunk(xs + 16 * l32, xc);
  float tot[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = h2f(t.s[i]) * dot16_i8(t.c[i], xc, 0.0f);
    v = lemoq_attn::group_sum_lanes<16>(v, lane);  // every lane holds its 16-lane row's total
    tot[i][0] = lane_f(v, 0) + lane_f(v, 16);       // row 2i   (lanes 0-31)
    tot[i][1] = lane_f(v, 32) + lane_f(v, 48);      // row 2i+1 (lanes 32-63)
  }
  float out = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
      if (lane == 2 * i + hf) out = tot[i][hf];
  if (lane < MO_ROWS_WAVE) a.part[(int64_t)t.g * a.N + t.row0 + lane] = out;
}

// Block (x, g) of the standalone launch -> o_proj tile (rb, g).  Blocks are
// dispatched round-robin over the 8 XCDs (each with its own L2): linear block
// b goes to XCD b % 8.  With G = heads / 4 groups and R = N / 32 row blocks,
// when G divides 8 and R * G is a multiple of 8, the blocks of XCD c all take
// head group c % G, so each L2 fetches one group's 33 KB of split partials
// instead of every group's.
__device__ __forceinline__ void oproj_tile_of_block(int& g, int& rb) {
  const int G = gridDim.y, R = gridDim.x;
  const int b = blockIdx.x + R * blockIdx.y;
  g = blockIdx.y;
  rb = blockIdx.x;
  if (8 % G == 0 && (R * G) % 8 == 0) {
    const int xcd = b % 8, k = b / 8;  // k-th block on this XCD, k < R * G / 8
    const int per = 8 / G;             // XCDs per head group
    g = xcd % G;
    rb = (xcd / G) + per * k;          // XCDs of one group interleave its row blocks
  }
}

struct RouterResidArgs {
  const float* part;  // (NP, H) o_proj partial sums
  const uint16_t* h;  // (H) residual stream before o_proj
  const uint16_t* norm_w;
  float eps;
  int H;
  const uint16_t* rw;  // (E, H) fp16 router weight
  int E;
  uint16_t* h_out;   // (H) h' = fp16(fp16(o) + h), written by block 0
  uint16_t* xn_out;  // (H) RMSNorm(h'), written by block 0 when non-null
  uint16_t* logits;  // (E)
};

__device__ __forceinline__ float f32_of(uint32_t v) { return __builtin_bit_cast(float, v); }

// One wave per expert row (4 per block).  Every block rebuilds h' and its
// norm: thread t owns the 8 values at (256 i + t) * 8 for i < H / 2048; the
// sum of squares is one 4-wave reduction through LDS, and the normalised row
// is staged in LDS for the waves' dots (lane l reads [1024 j + 16 l, +16),
// the order of lemoq_router_logits).  Loads first: router_issue loads the
// wave's router row and the block's slices of h and of the norm weight (none
// of which depends on the o_proj partials), router_finish the partials.
template <int KCH>
struct RouterPre {
  static constexpr int NV = KCH / 2;
  XRaw<KCH> wr;
  u32x4 hv[NV], nv[NV];
};

template <int KCH>
__device__ __forceinline__ void router_issue(const RouterResidArgs& a, int blk, RouterPre<KCH>& p) {
  constexpr int NV = KCH / 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blk * 4 + wave;
  const int ec = e < a.E ? e : a.E - 1;
  x_issue<KCH, true>(p.wr, a.rw + (int64_t)ec * a.H, a.H, true, lane);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int off = (i * 256 + threadIdx.x) * 8;
    p.hv[i] = *reinterpret_cast<const u32x4*>(a.h + off);
    p.nv[i] = *reinterpret_cast<const u32x4*>(a.norm_w + off);
  }
}

// o = fp16(sum of the NP partial rows), h' = fp16(o + h), the norm and the
// router logits of block `blk`'s 4 experts.  xs: KCH * 1024 fp16 of LDS, red: 4
// floats.
template <int KCH, int NP>
__device__ __forceinline__ void router_finish(const RouterResidArgs& a, int blk, const RouterPre<KCH>& p,
                                              uint16_t* xs, float* red) {
  constexpr int NV = KCH / 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blk * 4 + wave;
  u32x4 pv[NV][NP][2];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int off = (i * 256 + threadIdx.x) * 8;
#pragma unroll
    for (int g = 0; g < NP; ++g) {
      pv[i][g][0] = *reinterpret_cast<const u32x4*>(a.part + (int64_t)g * a.H + off);
      pv[i][g][1] = *reinterpret_cast<const u32x4*>(a.part + (int64_t)g * a.H + off + 4);
    }
  }
  LEMOQ_LOADS_ISSUED();

  uint32_t hm[NV][4];
  float ssq = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float sum[8];
#pragma unroll
    for (int g = 0; g < NP; ++g) {
      const uint32_t w[8] = {pv[i][g][0].x, pv[i][g][0].y, pv[i][g][0].z, pv[i][g][0].w,
                             pv[i][g][1].x, pv[i][g][1].y, pv[i][g][1].z, pv[i][g][1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) sum[q] = g == 0 ? f32_of(w[q]) : sum[q] + f32_of(w[q]);
    }
    const uint32_t hw[4] = {p.hv[i].x, p.hv[i].y, p.hv[i].z, p.hv[i].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t lo = hadd_round(h2f(f2h(sum[2 * k])), (uint16_t)(hw[k] & 0xFFFFu));
      const uint16_t hi = hadd_round(h2f(f2h(sum[2 * k + 1])), (uint16_t)(hw[k] >> 16));
      const float x0 = h2f(lo), x1 = h2f(hi);
      ssq = fmaf(x0, x0, ssq);
      ssq = fmaf(x1, x1, ssq);
      hm[i][k] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
  }
  ssq = wave_sum(ssq);
  if (lane == 0) red[wave] = ssq;
  __syncthreads();
  const float rstd = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)a.H + a.eps);
  u32x4 xv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int off = (i * 256 + threadIdx.x) * 8;
    const uint32_t gw[4] = {p.nv[i].x, p.nv[i].y, p.nv[i].z, p.nv[i].w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t n0 = f2h(h2f((uint16_t)(hm[i][k] & 0xFFFFu)) * rstd);
      const uint16_t n1 = f2h(h2f((uint16_t)(hm[i][k] >> 16)) * rstd);
      const uint16_t y0 = f2h(h2f(n0) * h2f((uint16_t)(gw[k] & 0xFFFFu)));
      const uint16_t y1 = f2h(h2f(n1) * h2f((uint16_t)(gw[k] >> 16)));
      o[k] = (uint32_t)y0 | ((uint32_t)y1 << 16);
    }
    xv[i] = (u32x4){o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4*>(xs + off) = xv[i];
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const u32x4 xw4 = *reinterpret_cast<const u32x4*>(xs + 1024 * j + 16 * lane + 8 * q);
      const uint32_t ww[4] = {p.wr.v[j][q].x, p.wr.v[j][q].y, p.wr.v[j][q].z, p.wr.v[j][q].w};
      const uint32_t xw[4] = {xw4.x, xw4.y, xw4.z, xw4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(as_h2(ww[i]), as_h2(xw[i]), acc, false);
    }
  acc = wave_sum(acc);
  if (lane == 0 && e < a.E) a.logits[e] = f2h(acc);
  // Block 0's copies of h' and xn go last: a store waited on before the
  // norm would hold back block 0 (the memory counter also counts stores).
  if (blk == 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int off = (i * 256 + threadIdx.x) * 8;
      *reinterpret_cast<u32x4*>(a.h_out + off) = (u32x4){hm[i][0], hm[i][1], hm[i][2], hm[i][3]};
      if (a.xn_out) *reinterpret_cast<u32x4*>(a.xn_out + off) = xv[i];
    }
  }
}

}  // namespace lemoq_oproj
