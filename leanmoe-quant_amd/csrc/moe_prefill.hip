// MoE block for several tokens (prefill) on the matrix cores.
//
// The reference's multi-token MoE (_prefill_forward,
// src/lemoq/kernels/moe_static.py:329-371) loops over experts: for expert e it
// gathers the tokens routed to it (nonzero of top_i == e, token order), runs
// gu = x_e @ dequant(gate_up_e)^T and y = (silu(gate) * up) @ dequant(down_e)^T
// as fp16 F.linear calls, and index_adds y * w into a zero fp16 output, one
// expert after the other.  Here each expert's weights are read once by a
// grouped GEMM over all of its tokens, in four launches:
//
//  1. moe_sort: stable counting sort of the (token, slot) pairs by expert
//     (pairs of one expert stay in token order), the pairs' fp16 routing
//     weights (top_w.to(fp16), moe_static.py:281-283), and a table of
//     128-row tiles, each inside one expert's run of pairs.
//  2. moe_gate_up: act = fp16(fp16(silu(g)) * u) with g, u the fp16 outputs of
//     the gate and up rows (the reference's gu.chunk, act_fn(gate) * up);
//     gate and up columns n sit in the same lane, so the product is formed in
//     the GEMM epilogue.
//  3. moe_down: y = fp16(act @ w_down^T), then fp16(y * w) (the `y * w` of
//     the index_add), written to row token*top_k + slot.
//  4. moe_combine: out = 0; out = fp16(out + y_slot) over the token's slots
//     in ascending expert order (the order of the expert loop; a token meets
//     each expert at most once, so index_add_ adds one term per expert), then
//     fp16(residual + out) (HF's decoder-layer residual add).
//
// The weights dequantise to fp16(code * scale) as the reference's prefill
// does (dequant_*_expert(e, dtype=x.dtype), moe_grouped_quant.py:173-188).
#include "gemm_core.h"

namespace {

using namespace lemoq_gemm;

constexpr int TILE_ROWS = 128;    // rows of a tile (2 waves of 64 along M)
constexpr int MAX_PAIRS = 32768;  // T * top_k held as bytes in LDS by moe_sort
constexpr int MAX_EXPERTS = 255;  // expert ids are bytes; 255 marks an invalid id

// ---------------------------------------------------------------------------
// 1. sort.  One block of 1024 threads per expert; each block stages the ids
// in LDS as bytes and builds the full histogram (one private histogram per
// wave, then summed), derives its expert's pair offset and tile offset, writes
// its tiles, and places its pairs: each thread owns a contiguous run of
// pairs (read 4 ids at a time), counts its matches, and an exclusive scan over
// the threads gives the stable positions.  Block 0 writes expert_off and
// marks the unused tail of the tile table (expert -1).
// ---------------------------------------------------------------------------
constexpr int SORT_THREADS = 1024;
constexpr int SORT_WAVES = SORT_THREADS / 64;
constexpr int RUN4 = (MAX_PAIRS / 4 + SORT_THREADS - 1) / SORT_THREADS;  // words of 4 pairs per thread, at most

__global__ __launch_bounds__(SORT_THREADS) void moe_sort_kernel(const int64_t* __restrict__ top_i,
                                                                const float* __restrict__ top_w, int P,
                                                                int top_k, int E, int32_t* __restrict__ pair_tok,
                                                                int32_t* __restrict__ pair_src,
                                                                uint16_t* __restrict__ pair_w,
                                                                int32_t* __restrict__ expert_off,
                                                                int32_t* __restrict__ tiles, int max_tiles) {
  __shared__ __align__(16) uint8_t ids[MAX_PAIRS];
  __shared__ int whist[SORT_WAVES][256];
  __shared__ int hist[256];
  __shared__ int wave_tot[SORT_WAVES];
  __shared__ int ex_off[257], ex_toff[257];  // exclusive prefixes over the experts; [256] the totals
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int me = blockIdx.x;
  // Each thread owns a run of at most RUN4 words of 4 pairs (placement below).
  const int P4 = (P + 3) / 4;
  const int chunk4 = (P4 + SORT_THREADS - 1) / SORT_THREADS;
  const int beg4 = min(P4, tid * chunk4), end4 = min(P4, beg4 + chunk4);
  for (int i = lane; i < 256; i += 64) whist[wave][i] = 0;
  __syncthreads();
  // The ids are loaded 8 per thread at a time (a load per loop trip would
  // make each of the thread's P / 1024 ids one more dependent memory round
  // trip).
  constexpr int IB = 8;
  for (int j0 = 0; SORT_THREADS * j0 < P; j0 += IB) {
    int64_t ev[IB];
#pragma unroll
    for (int j = 0; j < IB; ++j) {
      const int p = tid + SORT_THREADS * (j0 + j);
      ev[j] = p < P ? top_i[p] : -1;
    }
#pragma unroll
    for (int j = 0; j < IB; ++j) {
      const int p = tid + SORT_THREADS * (j0 + j);
      if (p >= P) break;
      const bool ok = ev[j] >= 0 && ev[j] < E;
      ids[p] = ok ? (uint8_t)ev[j] : (uint8_t)255;
      if (ok) atomicAdd(&whist[wave][(int)ev[j]], 1);
    }
  }
  // pad the byte array to a multiple of 4 with invalid ids
  if (tid < 4 && P + tid < ((P + 3) & ~3)) ids[P + tid] = 255;
  __syncthreads();
  if (tid < 256) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < SORT_WAVES; ++w) c += whist[w][tid];
    hist[tid] = c;
  }
  __syncthreads();
  // Exclusive prefix sums over the experts of the pair counts and of the tile
  // counts, by wave 0 (lane l owns experts 4l .. 4l + 3): one wave scan
  // instead of a serial loop over the experts.
  if (wave == 0) {
    int c[4], tc[4], cs = 0, ts = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * lane + j;
      c[j] = e < E ? hist[e] : 0;
      tc[j] = (c[j] + TILE_ROWS - 1) / TILE_ROWS;
      cs += c[j];
      ts += tc[j];
    }
    int ci = cs, ti = ts;  // inclusive scans over the lanes
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int a = __shfl_up(ci, d, 64), b = __shfl_up(ti, d, 64);
      if (lane >= d) ci += a, ti += b;
    }
    int o = ci - cs, t = ti - ts;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ex_off[4 * lane + j] = o;
      ex_toff[4 * lane + j] = t;
      o += c[j];
      t += tc[j];
    }
    if (lane == 63) ex_off[256] = o, ex_toff[256] = t;  // totals
  }
  __syncthreads();
  if (me == 0) {
    for (int e = tid; e <= E; e += SORT_THREADS) expert_off[e] = ex_off[e < E ? e : 256];
    for (int i = ex_toff[256] + tid; i < max_tiles; i += SORT_THREADS) tiles[4 * i] = -1;
  }
  const int cnt = hist[me], off = ex_off[me];
  const int ntiles = (cnt + TILE_ROWS - 1) / TILE_ROWS;
  for (int i = tid; i < ntiles; i += SORT_THREADS) {
    int32_t* t = tiles + 4 * (ex_toff[me] + i);
    t[0] = me;
    t[1] = off + i * TILE_ROWS;
    t[2] = off + min(cnt, (i + 1) * TILE_ROWS);
    t[3] = 0;
  }
  const uint32_t* ids4 = reinterpret_cast<const uint32_t*>(ids);
  const uint32_t mev = (uint32_t)me * 0x01010101u;
  int c = 0;
#pragma unroll
  for (int i = 0; i < RUN4; ++i) {
    if (beg4 + i >= end4) break;
    const uint32_t x = ids4[beg4 + i] ^ mev;  // a zero byte marks a match
#pragma unroll
    for (int b = 0; b < 4; ++b) c += ((x >> (8 * b)) & 0xFFu) == 0u;
  }
  int incl = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(incl, d, 64);
    if (lane >= d) incl += t;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int pos = off + incl - c;
  for (int w = 0; w < wave; ++w) pos += wave_tot[w];
  // The routing weights of the run's matches are all loaded before the first
  // store (one load per matching pair, issued back to back).
  uint32_t xm[RUN4];
  float wrun[4 * RUN4];
#pragma unroll
  for (int i = 0; i < RUN4; ++i) {
    xm[i] = beg4 + i < end4 ? ids4[beg4 + i] ^ mev : 0xFFFFFFFFu;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const bool hit = ((xm[i] >> (8 * b)) & 0xFFu) == 0u;
      wrun[4 * i + b] = hit ? top_w[4 * (beg4 + i) + b] : 0.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < RUN4; ++i) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (((xm[i] >> (8 * b)) & 0xFFu) != 0u) continue;
      const int p = 4 * (beg4 + i) + b;
      pair_tok[pos] = p / top_k;
      pair_src[pos] = p;
      pair_w[pos] = f2h(wrun[4 * i + b]);
      ++pos;
    }
  }
}

struct GroupedArgs {
  const uint16_t* x;        // gate_up: hidden rows (T, H); down: act rows (P, F)
  const int32_t* pair_tok;  // gate_up: token of each sorted pair
  const int32_t* pair_src;  // down: output row of each sorted pair
  const uint16_t* pair_w;   // down: fp16 routing weight of each sorted pair
  const int32_t* tiles;     // (max_tiles, 4): expert, row begin, row end, 0
  const int8_t* codes;      // (E, rows_per_expert, K)
  const uint16_t* scale;    // (E, rows_per_expert, K / group)
  int64_t K;                // reduction width (H for gate_up, F for down)
  int64_t N;                // output columns (F for gate_up, H for down)
  int group;
  uint16_t* y;              // gate_up: act (P, F); down: (T * top_k, H)
};

// Grouped GEMM blocks: a 1-D grid over (column block nb, tile mt) numbered
// nb-major, so consecutive blocks take consecutive tiles of the same column
// block (usually the same expert, i.e. the same weight tile), and each XCD
// takes a contiguous range of them.  Block tile 128 pairs x BN weight rows,
// 2 x WN waves of 64 x 64 (the stage pipeline of gemm_core.h).
#ifndef LEMOQ_MOE_WN
#define LEMOQ_MOE_WN 4  // column waves per grouped block (2: 128 weight rows, 4: 256)
#endif
constexpr int MOE_WN = LEMOQ_MOE_WN;
constexpr int64_t kSmallTiles = 16;  // tile tables this small run 64-row blocks (WN = 1)
template <int WN>
using GTile = Tile<128, 64 * WN, 2, WN>;

__device__ __forceinline__ bool grouped_tile(const GroupedArgs& a, int64_t ncol_blocks, int64_t max_tiles,
                                             int64_t& nb, int& e, int64_t& rs, int64_t& re) {
  const int64_t lin = xcd_tile(blockIdx.x, ncol_blocks * max_tiles);
  nb = lin / max_tiles;
  const int32_t* tl = a.tiles + 4 * (lin % max_tiles);
  e = tl[0];
  rs = tl[1];
  re = tl[2];
  return e >= 0;
}

// 2. gate_up: the block's 64 WN weight rows are AC = 32 WN gate rows (act
// columns n0 .. n0 + AC - 1) and the AC matching up rows, so wave (wm, wn)
// pairs gate rows 32 wn .. 32 wn + 31 (fragment 0) with the same up rows
// (fragment 1).
template <int WN>
__global__ __launch_bounds__(128 * WN) void moe_gate_up_kernel(const GroupedArgs a, int64_t max_tiles) {
  using TL = GTile<WN>;
  constexpr int AC = 32 * WN;  // act columns per block
  __shared__ __align__(16) uint16_t lds[TL::LDS_ELEMS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int64_t F = a.N;
  int64_t nb, rs, re;
  int e;
  if (!grouped_tile(a, (F + AC - 1) / AC, max_tiles, nb, e, rs, re)) return;  // block-uniform
  const int64_t n0 = nb * AC;
  Sources<TL, true> src;
#pragma unroll
  for (int i = 0; i < TL::A_CH; ++i) {
    int64_t m = rs + TL::a_row(t, i);
    m = m < re ? m : re - 1;
    src.a[i] = a.x + (int64_t)a.pair_tok[m] * a.K + TL::a_col(t, i);
  }
  const int64_t ng = a.K / a.group;
#pragma unroll
  for (int i = 0; i < TL::B8_CH; ++i) {
    const int r = TL::b8_row(t, i);
    int64_t n = n0 + (r & (AC - 1));
    n = n < F ? n : F - 1;
    const int64_t row = (int64_t)e * 2 * F + (r < AC ? n : F + n);
    src.bc[i] = a.codes + row * a.K + TL::b8_col(t, i);
    src.bs[i] = a.scale + row * ng;
  }
  const int wm = wave / WN, wn = wave % WN;
  const int b_row0[2] = {32 * wn, AC + 32 * wn};
  Acc<2, 2> acc;
  block_mainloop2<TL, true>(acc, src, a.K, a.group, lds, 64 * wm, b_row0);
  const int64_t n = n0 + 32 * wn + l32;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t m = rs + 64 * wm + 32 * i + acc_row(r, half);
      if (m >= re || n >= F) continue;
      const float g = h2f(f2h(acc.v[i][0][r]));
      const float u = h2f(f2h(acc.v[i][1][r]));
      const float sg = h2f(f2h(g / (1.0f + expf(-g))));
      a.y[m * F + n] = f2h(sg * u);
    }
}

// 3. down: 128 pairs x 64 WN hidden columns per block.  The epilogue goes
// through LDS: the waves write fp16(acc) into the (then idle) stage buffers
// as a 128 x 64 WN row-major tile, and the block writes each pair's row
// segment with 16-byte stores, scaled by its routing weight on the way out:
// fp16(fp16(y) * w), the same two roundings as per element.  The pair's
// output row and weight are loaded before the K loop (threads 0..127, one
// pair each) and parked in LDS for the epilogue.
template <int WN>
__global__ __launch_bounds__(128 * WN) void moe_down_kernel(const GroupedArgs a, int64_t max_tiles) {
  using TL = GTile<WN>;
  constexpr int NC = 64 * WN;       // output columns per block
  constexpr int OP = NC + 8;        // output tile pitch in LDS (fp16)
  constexpr int CPR = NC / 8;       // 16-byte chunks per output row
  constexpr int RPI = TL::NT / CPR; // rows written per pass of the block
  static_assert(TILE_ROWS * OP <= TL::LDS_ELEMS && TL::NT % CPR == 0, "down output tile");
  __shared__ __align__(16) uint16_t lds[TL::LDS_ELEMS];
  __shared__ int32_t row_dst[TILE_ROWS];
  __shared__ float row_w[TILE_ROWS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int64_t H = a.N;
  int64_t nb, rs, re;
  int e;
  if (!grouped_tile(a, (H + NC - 1) / NC, max_tiles, nb, e, rs, re)) return;  // block-uniform
  const int64_t n0 = nb * NC;
  const int rows = (int)(re - rs);  // 1 .. TILE_ROWS
  int32_t my_dst = 0;
  uint16_t my_w = 0;
  if (t < rows) {
    my_dst = a.pair_src[rs + t];
    my_w = a.pair_w[rs + t];
  }
  Sources<TL, true> src;
#pragma unroll
  for (int i = 0; i < TL::A_CH; ++i) {
    int64_t m = rs + TL::a_row(t, i);
    m = m < re ? m : re - 1;
    src.a[i] = a.x + m * a.K + TL::a_col(t, i);
  }
  const int64_t ng = a.K / a.group;
#pragma unroll
  for (int i = 0; i < TL::B8_CH; ++i) {
    int64_t n = n0 + TL::b8_row(t, i);
    n = n < H ? n : H - 1;
    const int64_t row = (int64_t)e * H + n;
    src.bc[i] = a.codes + row * a.K + TL::b8_col(t, i);
    src.bs[i] = a.scale + row * ng;
  }
  const int wm = wave / WN, wn = wave % WN;
  const int b_row0[2] = {64 * wn, 64 * wn + 32};
  Acc<2, 2> acc;
  block_mainloop2<TL, true>(acc, src, a.K, a.group, lds, 64 * wm, b_row0);
  __syncthreads();  // every wave has read its last stage from LDS
  if (t < TILE_ROWS) {
    row_dst[t] = my_dst;
    row_w[t] = h2f(my_w);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        lds[(64 * wm + 32 * i + acc_row(r, half)) * OP + 64 * wn + 32 * j + l32] = f2h(acc.v[i][j][r]);
  __syncthreads();
  const int c8 = (t % CPR) * 8;
  const int64_t n = n0 + c8;
  if (n >= H) return;  // N % 32 == 0: a chunk is wholly inside or outside
  for (int row = t / CPR; row < rows; row += RPI) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(lds + row * OP + c8);
    const float w = row_w[row];
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint16_t lo = f2h(h2f((uint16_t)(in[q] & 0xFFFFu)) * w);
      const uint16_t hi = f2h(h2f((uint16_t)(in[q] >> 16)) * w);
      o[q] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *reinterpret_cast<u32x4*>(a.y + (int64_t)row_dst[row] * H + n) = (u32x4){o[0], o[1], o[2], o[3]};
  }
}

// 4. combine: one block per token, 8 columns per thread.  The slot loop has a
// fixed trip count of 8 (slots past top_k read slot 0 and are not added), so
// all of a thread's loads are issued before the first add.  (Loading the
// slots in slot order before the ids arrive, then reordering them through a
// 32 KB LDS stage, was slower: the stage caps the blocks per CU.)  NORM: the
// block keeps its output row in LDS and writes the next layer's input
// RMSNorm of it with the norm kernel's own row function (rmsnorm_chunks), so
// xn is bit-identical to a separate norm launch.  (Holding the row in
// registers instead raised the kernel to 93 registers and cost occupancy.)
constexpr int kCombineNormMaxH = 8192;

template <bool NORM>
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ y,
                                                          const int64_t* __restrict__ top_i,
                                                          int top_k, int64_t H,
                                                          const uint16_t* __restrict__ resid,
                                                          uint16_t* __restrict__ out,
                                                          const uint16_t* __restrict__ norm_w, float eps,
                                                          uint16_t* __restrict__ xn) {
  __shared__ __align__(16) uint16_t row[NORM ? kCombineNormMaxH : 8];
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  int64_t ids[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) ids[s] = top_i[t * top_k + (s < top_k ? s : 0)];
  // slot of rank o in ascending expert id (slot order among equal ids), with
  // static indexing only (a runtime index into ids would place it in scratch)
  int rank[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    int r = 0;
#pragma unroll
    for (int s2 = 0; s2 < 8; ++s2) r += (s2 < top_k && (ids[s2] < ids[s] || (ids[s2] == ids[s] && s2 < s))) ? 1 : 0;
    rank[s] = r;
  }
  int order[8];
#pragma unroll
  for (int o = 0; o < 8; ++o) {
    int slot = 0;
#pragma unroll
    for (int s = 0; s < 8; ++s) slot = (s < top_k && rank[s] == o) ? s : slot;
    order[o] = slot;
  }
  for (int64_t c = (int64_t)threadIdx.x * 8; c < H; c += 256 * 8) {
    u32x4 v[8];
#pragma unroll
    for (int o = 0; o < 8; ++o) v[o] = *reinterpret_cast<const u32x4*>(y + (t * top_k + order[o]) * H + c);
    u32x4 r = (u32x4){0u, 0u, 0u, 0u};
    if (resid) r = *reinterpret_cast<const u32x4*>(resid + t * H + c);
    LEMOQ_LOADS_ISSUED();
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int o = 0; o < 8; ++o) {
      const uint32_t w[4] = {v[o].x, v[o].y, v[o].z, v[o].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = h2f(f2h(acc[2 * i] + h2f((uint16_t)(w[i] & 0xFFFFu))));
        const float hi = h2f(f2h(acc[2 * i + 1] + h2f((uint16_t)(w[i] >> 16))));
        acc[2 * i] = o < top_k ? lo : acc[2 * i];
        acc[2 * i + 1] = o < top_k ? hi : acc[2 * i + 1];
      }
    }
    uint32_t ow[4];
    const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = resid ? hadd_round(acc[2 * i], (uint16_t)(rw[i] & 0xFFFFu)) : f2h(acc[2 * i]);
      const uint16_t hi = resid ? hadd_round(acc[2 * i + 1], (uint16_t)(rw[i] >> 16)) : f2h(acc[2 * i + 1]);
      ow[i] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    const u32x4 o4 = (u32x4){ow[0], ow[1], ow[2], ow[3]};
    *reinterpret_cast<u32x4*>(out + t * H + c) = o4;
    if constexpr (NORM) *reinterpret_cast<u32x4*>(row + c) = o4;
  }
  if constexpr (NORM) {
    // each thread reads back only the chunks it wrote: no barrier needed
    u32x4 ox[RN_CHUNKS];
    rmsnorm_load_chunks(row, (int)H, ox);
    rmsnorm_chunks(ox, (int)H, norm_w, eps, xn + t * H, red);
  }
}

bool grouped_shape_ok(int64_t K, int64_t N, int64_t group) {
  return K > 0 && N > 0 && K % 64 == 0 && N % 32 == 0 && group > 0 && group % 64 == 0 && K % group == 0 &&
         N <= (1LL << 24);
}

}  // namespace

extern "C" int64_t lemoq_moe_prefill_max_tiles(int64_t pairs, int64_t E) {
  return pairs / TILE_ROWS + E;
}

extern "C" int lemoq_moe_prefill_sort(const int64_t* top_i, const float* top_w, int64_t T, int64_t top_k,
                                      int64_t E, int32_t* pair_tok, int32_t* pair_src, uint16_t* pair_w,
                                      int32_t* expert_off, int32_t* tiles, int64_t max_tiles, void* stream) {
  if (!top_i || !top_w || !pair_tok || !pair_src || !pair_w || !expert_off || !tiles) return LEMOQ_ERR_NULL;
  if (T <= 0 || top_k <= 0 || top_k > 8 || E <= 0 || E > MAX_EXPERTS || top_k > E) return LEMOQ_ERR_SHAPE;
  if (T * top_k > MAX_PAIRS) return LEMOQ_ERR_UNSUPPORTED;
  if (max_tiles < lemoq_moe_prefill_max_tiles(T * top_k, E) || max_tiles > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(moe_sort_kernel, dim3((unsigned)E), dim3(SORT_THREADS), 0, lemoq_stream(stream), top_i, top_w,
                     (int)(T * top_k), (int)top_k, (int)E, pair_tok, pair_src, pair_w, expert_off, tiles,
                     (int)max_tiles);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_moe_prefill_gate_up(const uint16_t* x, int64_t H, const int32_t* pair_tok,
                                         const int32_t* tiles, int64_t max_tiles, const int8_t* gu_codes,
                                         const uint16_t* gu_scale, int64_t F, int64_t group, uint16_t* act,
                                         void* stream) {
  if (!x || !pair_tok || !tiles || !gu_codes || !gu_scale || !act) return LEMOQ_ERR_NULL;
  if (!grouped_shape_ok(H, F, group) || max_tiles <= 0 || max_tiles > (1LL << 20)) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(x) || !lemoq_aligned16(gu_codes)) return LEMOQ_ERR_ALIGN;
  GroupedArgs a{};
  a.x = x; a.pair_tok = pair_tok; a.tiles = tiles; a.codes = gu_codes; a.scale = gu_scale;
  a.K = H; a.N = F; a.group = (int)group; a.y = act;
  // A table of at most 16 tiles (e.g. one token's top_k experts, passed with
  // max_tiles = top_k) leaves most CUs idle with 256 weight rows per block:
  // 64 rows per block there (the same arithmetic per element).
  if (max_tiles <= kSmallTiles) {
    const int64_t blocks = ((F + 31) / 32) * max_tiles;
    hipLaunchKernelGGL(moe_gate_up_kernel<1>, dim3((unsigned)blocks), dim3(128), 0, lemoq_stream(stream), a,
                       max_tiles);
    LEMOQ_CHECK_LAUNCH();
  }
  const int64_t blocks = ((F + 32 * MOE_WN - 1) / (32 * MOE_WN)) * max_tiles;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(moe_gate_up_kernel<MOE_WN>, dim3((unsigned)blocks), dim3(128 * MOE_WN), 0,
                     lemoq_stream(stream), a, max_tiles);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_moe_prefill_down(const uint16_t* act, int64_t F, const int32_t* pair_src,
                                      const uint16_t* pair_w, const int32_t* tiles, int64_t max_tiles,
                                      const int8_t* dn_codes, const uint16_t* dn_scale, int64_t H,
                                      int64_t group, uint16_t* y, void* stream) {
  if (!act || !pair_src || !pair_w || !tiles || !dn_codes || !dn_scale || !y) return LEMOQ_ERR_NULL;
  if (!grouped_shape_ok(F, H, group) || max_tiles <= 0 || max_tiles > (1LL << 20)) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(act) || !lemoq_aligned16(dn_codes) || !lemoq_aligned16(y)) return LEMOQ_ERR_ALIGN;
  GroupedArgs a{};
  a.x = act; a.pair_src = pair_src; a.pair_w = pair_w; a.tiles = tiles; a.codes = dn_codes;
  a.scale = dn_scale; a.K = F; a.N = H; a.group = (int)group; a.y = y;
  if (max_tiles <= kSmallTiles) {  // as in lemoq_moe_prefill_gate_up
    const int64_t blocks = ((H + 63) / 64) * max_tiles;
    hipLaunchKernelGGL(moe_down_kernel<1>, dim3((unsigned)blocks), dim3(128), 0, lemoq_stream(stream), a,
                       max_tiles);
    LEMOQ_CHECK_LAUNCH();
  }
  const int64_t blocks = ((H + 64 * MOE_WN - 1) / (64 * MOE_WN)) * max_tiles;
  if (blocks > 0x7fffffffLL) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(moe_down_kernel<MOE_WN>, dim3((unsigned)blocks), dim3(128 * MOE_WN), 0,
                     lemoq_stream(stream), a, max_tiles);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_moe_prefill_combine(const uint16_t* y, const int64_t* top_i, int64_t T, int64_t top_k,
                                         int64_t H, const uint16_t* residual, uint16_t* out, void* stream) {
  if (!y || !top_i || !out) return LEMOQ_ERR_NULL;
  if (T <= 0 || T > 0x7fffffffLL || top_k <= 0 || top_k > 8 || H <= 0 || H % 8 != 0) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(y) || !lemoq_aligned16(out) || (residual && !lemoq_aligned16(residual)))
    return LEMOQ_ERR_ALIGN;
  hipLaunchKernelGGL(moe_combine_kernel<false>, dim3((unsigned)T), dim3(256), 0, lemoq_stream(stream), y, top_i,
                     (int)top_k, H, residual, out, nullptr, 0.0f, nullptr);
  LEMOQ_CHECK_LAUNCH();
}

extern "C" int lemoq_moe_prefill_combine_norm(const uint16_t* y, const int64_t* top_i, int64_t T, int64_t top_k,
                                              int64_t H, const uint16_t* residual, uint16_t* out,
                                              const uint16_t* norm_w, float eps, uint16_t* xn_out, void* stream) {
  if (!y || !top_i || !out || !norm_w || !xn_out) return LEMOQ_ERR_NULL;
  if (T <= 0 || T > 0x7fffffffLL || top_k <= 0 || top_k > 8 || H <= 0 || H % 8 != 0 || H > kCombineNormMaxH)
    return LEMOQ_ERR_SHAPE;
  // the row norm reads norm_w and writes xn_out in 16-byte chunks too
  if (!lemoq_aligned16(y) || !lemoq_aligned16(out) || (residual && !lemoq_aligned16(residual)) ||
      !lemoq_aligned16(norm_w) || !lemoq_aligned16(xn_out))
    return LEMOQ_ERR_ALIGN;
  // xn_out must not overlap the rows the block reads (y, the residual) or writes (out)
  const uintptr_t xa = (uintptr_t)xn_out, xb = xa + (uintptr_t)(T * H * 2);
  const uintptr_t oa = (uintptr_t)out, ob = oa + (uintptr_t)(T * H * 2);
  if (xa < ob && oa < xb) return LEMOQ_ERR_SHAPE;
  if (residual) {
    const uintptr_t ra = (uintptr_t)residual, rb = ra + (uintptr_t)(T * H * 2);
    if (xa < rb && ra < xb) return LEMOQ_ERR_SHAPE;
  }
  const uintptr_t ya = (uintptr_t)y, yb = ya + (uintptr_t)(T * top_k * H * 2);
  if (xa < yb && ya < xb) return LEMOQ_ERR_SHAPE;
  hipLaunchKernelGGL(moe_combine_kernel<true>, dim3((unsigned)T), dim3(256), 0, lemoq_stream(stream), y, top_i,
                     (int)top_k, H, residual, out, norm_w, eps, xn_out);
  LEMOQ_CHECK_LAUNCH();
}
