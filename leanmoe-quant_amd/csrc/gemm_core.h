// Matrix-core main loop shared by the multi-token (prefill) GEMMs.
//
// A block of WM x WN waves computes a BM x BN tile of Y = X W^T with
// v_mfma_f32_32x32x16_f16; X rows fp16, W rows either w8 (int8 codes + fp16
// per-group scales, dequantised to fp16(code * scale) once per block as the
// tile is written to LDS) or fp16.  K advances in stages of 64: the global
// loads of a stage are issued into registers two stages ahead, then written
// to the other half of a double-buffered LDS tile while the current stage's
// matrix ops run; one barrier per stage.  Loads are never under a branch: the
// prefetches past the last stage re-read the last stage (clamped k).
//
// Operand layout of v_mfma_f32_32x32x16_f16 (verified on the device): lane l
// holds row (A) / column (B) l % 32 and 8 k-values of the lane half l / 32;
// accumulator register r of lane l is element (8*(r/4) + 4*(l/32) + r%4,
// l % 32).  The sum over k does not depend on which k-values a lane half
// holds as long as A and B agree, so each lane reads 16 consecutive k of a
// 32-wide chunk (two 16-byte LDS reads) and feeds two instructions: half h
// takes 16h + [0, 8) in the first and 16h + [8, 16) in the second.
#pragma once

#include "common.h"

namespace lemoq_gemm {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;            // k per stage
constexpr int LDS_PITCH = BK + 8; // fp16 per LDS row (16-byte pad)

__device__ __forceinline__ h8v h8_of(const u32x4 v) { return __builtin_bit_cast(h8v, v); }

// 16 int8 codes (k order) -> two u32x4 of fp16(code * s): the code becomes an
// exact fp16 through (1024 + (code + 128)) - 1152, and one fp16 multiply
// rounds the exact product once (the fp32 product code * scale is exact, so
// this equals rounding it to fp16).
__device__ __forceinline__ void dequant16(const u32x4 c, uint32_t s2, u32x4& lo, u32x4& hi) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  const f16x2 sc = as_h2(s2);
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t t = w[i] ^ 0x80808080u;
    const uint32_t p01 = __builtin_amdgcn_perm(0x64646464u, t, 0x04010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(0x64646464u, t, 0x04030402u);
    o[2 * i] = __builtin_bit_cast(uint32_t, (as_h2(p01) - bias) * sc);
    o[2 * i + 1] = __builtin_bit_cast(uint32_t, (as_h2(p23) - bias) * sc);
  }
  lo = (u32x4){o[0], o[1], o[2], o[3]};
  hi = (u32x4){o[4], o[5], o[6], o[7]};
}

// Tile geometry of a BM x BN block computed by WM x WN waves (each wave a
// (BM / WM) x (BN / WN) sub-tile of 32 x 32 fragments).  Every thread of the
// block stages A_CH 16-byte A chunks and B8_CH (w8) or B16_CH (fp16) B
// chunks per stage.
template <int BM_, int BN_, int WM_ = 2, int WN_ = 2>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int NT = 64 * WM * WN;                 // threads per block
  static constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
  static constexpr int A_CH = BM * (BK / 8) / NT;   // 16-byte A chunks per thread per stage
  static constexpr int B16_CH = BN * (BK / 8) / NT; // fp16 B chunks per thread
  static constexpr int B8_CH = BN * (BK / 16) / NT; // w8 B chunks (16 codes) per thread
  static constexpr int LDS_HALF = (BM + BN) * LDS_PITCH;  // fp16 per buffer
  static constexpr int LDS_ELEMS = 2 * LDS_HALF;
  static_assert(FM >= 1 && FN >= 1 && A_CH >= 1 && B8_CH >= 1 && BM * (BK / 8) % NT == 0 &&
                    BN * (BK / 16) % NT == 0,
                "tile sizes");
  // Thread t's A chunk i: tile row (t + NT i) / 8, column 8 * ((t + NT i) % 8).
  __device__ static int a_row(int t, int i) { return (t + NT * i) >> 3; }
  __device__ static int a_col(int t, int i) { return 8 * ((t + NT * i) & 7); }
  __device__ static int b16_row(int t, int i) { return (t + NT * i) >> 3; }
  __device__ static int b16_col(int t, int i) { return 8 * ((t + NT * i) & 7); }
  // w8 chunk: 16 codes; tile row (t + NT i) / 4, column 16 * ((t + NT i) % 4).
  __device__ static int b8_row(int t, int i) { return (t + NT * i) >> 2; }
  __device__ static int b8_col(int t, int i) { return 16 * ((t + NT * i) & 3); }
};

template <int FM, int FN>
struct Acc {
  f32x16 v[FM][FN];
};

// Per-thread sources of one block: A chunk pointers (row start + column) and
// B chunk pointers (codes and the row's scales, or fp16 weights).
template <class TL, bool W8>
struct Sources {
  const uint16_t* a[TL::A_CH];
  const int8_t* bc[W8 ? TL::B8_CH : 1];
  const uint16_t* bs[W8 ? TL::B8_CH : 1];
  const uint16_t* bw[W8 ? 1 : TL::B16_CH];
};

template <class TL, bool W8>
struct Staged {
  u32x4 a[TL::A_CH];
  u32x4 b[W8 ? TL::B8_CH : TL::B16_CH];
  uint16_t s[W8 ? TL::B8_CH : 1];
};

// Loads of the stage at k0; sidx = k0 / group is the index of its scale
// (group % BK == 0, so one scale covers each 16-code chunk of the stage).
template <class TL, bool W8>
__device__ __forceinline__ void stage_load(Staged<TL, W8>& st, const Sources<TL, W8>& src, int64_t k0,
                                           int sidx) {
#pragma unroll
  for (int i = 0; i < TL::A_CH; ++i) st.a[i] = *reinterpret_cast<const u32x4*>(src.a[i] + k0);
  if constexpr (W8) {
#pragma unroll
    for (int i = 0; i < TL::B8_CH; ++i) {
      st.b[i] = *reinterpret_cast<const u32x4*>(src.bc[i] + k0);
      st.s[i] = src.bs[i][sidx];
    }
  } else {
#pragma unroll
    for (int i = 0; i < TL::B16_CH; ++i) st.b[i] = *reinterpret_cast<const u32x4*>(src.bw[i] + k0);
  }
}

template <class TL, bool W8>
__device__ __forceinline__ void stage_store(const Staged<TL, W8>& st, uint16_t* buf, int t) {
  uint16_t* As = buf;
  uint16_t* Bs = buf + TL::BM * LDS_PITCH;
#pragma unroll
  for (int i = 0; i < TL::A_CH; ++i)
    *reinterpret_cast<u32x4*>(As + TL::a_row(t, i) * LDS_PITCH + TL::a_col(t, i)) = st.a[i];
  if constexpr (W8) {
#pragma unroll
    for (int i = 0; i < TL::B8_CH; ++i) {
      u32x4 lo, hi;
      dequant16(st.b[i], (uint32_t)st.s[i] * 0x10001u, lo, hi);
      uint16_t* d = Bs + TL::b8_row(t, i) * LDS_PITCH + TL::b8_col(t, i);
      *reinterpret_cast<u32x4*>(d) = lo;
      *reinterpret_cast<u32x4*>(d + 8) = hi;
    }
  } else {
#pragma unroll
    for (int i = 0; i < TL::B16_CH; ++i)
      *reinterpret_cast<u32x4*>(Bs + TL::b16_row(t, i) * LDS_PITCH + TL::b16_col(t, i)) = st.b[i];
  }
}

// A wave's fragments of one stage: for each 32-k chunk c, A fragments at
// tile rows a_row0 + 32 i and B fragments at tile rows b_row0[j], two 16-byte
// LDS reads each.
template <class TL>
struct Frags {
  u32x4 a[BK / 32][TL::FM][2], b[BK / 32][TL::FN][2];
};

template <class TL>
__device__ __forceinline__ void stage_frags(Frags<TL>& f, const uint16_t* buf, int a_row0,
                                            const int (&b_row0)[TL::FN], int l32, int half) {
  const uint16_t* As = buf;
  const uint16_t* Bs = buf + TL::BM * LDS_PITCH;
#pragma unroll
  for (int c = 0; c < BK / 32; ++c) {
#pragma unroll
    for (int i = 0; i < TL::FM; ++i) {
      const uint16_t* p = As + (a_row0 + 32 * i + l32) * LDS_PITCH + 32 * c + 16 * half;
      f.a[c][i][0] = *reinterpret_cast<const u32x4*>(p);
      f.a[c][i][1] = *reinterpret_cast<const u32x4*>(p + 8);
    }
#pragma unroll
    for (int j = 0; j < TL::FN; ++j) {
      const uint16_t* p = Bs + (b_row0[j] + l32) * LDS_PITCH + 32 * c + 16 * half;
      f.b[c][j][0] = *reinterpret_cast<const u32x4*>(p);
      f.b[c][j][1] = *reinterpret_cast<const u32x4*>(p + 8);
    }
  }
}

template <class TL>
__device__ __forceinline__ void stage_mfma(Acc<TL::FM, TL::FN>& acc, const Frags<TL>& f) {
#pragma unroll
  for (int c = 0; c < BK / 32; ++c)
#pragma unroll
    for (int i = 0; i < TL::FM; ++i)
#pragma unroll
      for (int j = 0; j < TL::FN; ++j) {
        acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of(f.a[c][i][0]), h8_of(f.b[c][j][0]), acc.v[i][j], 0, 0, 0);
        acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h8_of(f.a[c][i][1]), h8_of(f.b[c][j][1]), acc.v[i][j], 0, 0, 0);
      }
}

// Whole K loop of a block, global loads two stages ahead.  Stage s sits in
// one LDS buffer, the loads of stage s + 1 in one register set (issued a
// stage earlier) and those of stage s + 2 go into the other.  A stage body:
// the wave reads all its fragments of stage s from LDS, writes stage s + 1
// (dequantised) to the other buffer, issues the loads of stage s + 2, then
// runs its matrix ops; one barrier per stage.  With the fragment reads and
// the stores ahead of the matrix ops the compiler places the dequantisation
// and the LDS writes between the matrix ops, and the matrix ops no longer
// wait on fragment reads issued in the middle of the stage: the grouped
// gate/up GEMM at the ctx-4096 shape went from 435-480 to 405-440 us with
// bit-identical outputs.  Loads two stages ahead instead of one took the
// same GEMM from 412-530 to 393-417 us (gfx950, 8 waves, two per SIMD).
template <class TL, bool W8>
__device__ __forceinline__ void block_mainloop2(Acc<TL::FM, TL::FN>& acc, const Sources<TL, W8>& src,
                                                int64_t K, int group, uint16_t* lds, int a_row0,
                                                const int (&b_row0)[TL::FN]) {
  const int t = threadIdx.x, lane = t & 63;
  const int half = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int i = 0; i < TL::FM; ++i)
#pragma unroll
    for (int j = 0; j < TL::FN; ++j) acc.v[i][j] = (f32x16){};
  // The scale index of stage p is p / spg (spg = group / BK stages per scale
  // group), kept as a running count in scalar registers: a division in the
  // loop would cost about a hundred scalar instructions per stage.
  const int nst = (int)(K / BK);
  const int spg = W8 ? group / BK : 1;
  int gi = 0, gc = 0;  // scale index and stage within the group of the next stage loaded
  auto advance = [&]() {
    if (++gc == spg) gc = 0, ++gi;
  };
  const int last = nst - 1;
  const int last_sidx = W8 ? last / spg : 0;  // the clamped prefetch re-reads stage nst - 1
  Staged<TL, W8> s0, s1;
  stage_load<TL, W8>(s0, src, 0, 0);
  advance();  // stage 1
  stage_load<TL, W8>(s1, src, (int64_t)(1 < nst ? 1 : 0) * BK, 1 < nst ? gi : 0);
  advance();  // stage 2
  stage_store<TL, W8>(s0, lds, t);
  __syncthreads();
  for (int s = 0; s < nst; s += 2) {
    // stage s in LDS buffer 0, s1 holds stage s + 1
    {
      const bool more = s + 2 < nst;
      Frags<TL> f;
      stage_frags<TL>(f, lds, a_row0, b_row0, l32, half);
      stage_store<TL, W8>(s1, lds + TL::LDS_HALF, t);
      stage_load<TL, W8>(s0, src, (int64_t)(more ? s + 2 : last) * BK, more ? gi : last_sidx);
      advance();
      stage_mfma<TL>(acc, f);
      __syncthreads();
    }
    if (s + 1 >= nst) break;
    // stage s + 1 in LDS buffer 1, s0 holds stage s + 2
    {
      const bool more = s + 3 < nst;
      Frags<TL> f;
      stage_frags<TL>(f, lds + TL::LDS_HALF, a_row0, b_row0, l32, half);
      stage_store<TL, W8>(s0, lds, t);
      stage_load<TL, W8>(s1, src, (int64_t)(more ? s + 3 : last) * BK, more ? gi : last_sidx);
      advance();
      stage_mfma<TL>(acc, f);
      __syncthreads();
    }
  }
}

// Row (within the 32-row fragment) of accumulator register r in lane half `half`.
__device__ __forceinline__ int acc_row(int r, int half) { return 8 * (r / 4) + 4 * half + (r % 4); }

// Block index -> tile index so that the blocks of one XCD (dispatched
// round-robin over 8) take a contiguous range of tiles.
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t nblocks) {
  if (nblocks % 8 != 0) return b;
  return (b % 8) * (nblocks / 8) + b / 8;
}

}  // namespace lemoq_gemm
