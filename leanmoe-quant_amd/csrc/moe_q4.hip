// Grouped MoE GEMVs for one token on 4-bit symmetric experts: top_k of E
// experts, int4 codes packed two per byte (the even column in the low nibble)
// with per-group fp16 scales, fp32 accumulation.  The 4-bit branch of the
// reference's grouped kernels (_gate_up_act_kernel_q / _down_sum_kernel_q
// with BITS=4, src/lemoq/kernels/_grouped_triton.py:235-398, nibbles expanded
// by _expand_int4 :235-247) and of quantize_fused_experts(bits=4)
// (src/lemoq/kernels/moe_grouped_quant.py:191-244).
//
// Same structure and numerics as the 8-bit kernels (moe.hip): gate/up grid
// (ceil(F / (4R)), top_k), wave w of block b computes the R gate rows and the
// R matching up rows of expert ids[slot] and writes act = fp16(silu(g) * u)
// (the routed form takes the router's fp16 logits and routes in every block,
// as moe.hip's routed 8-bit kernel does);
// down grid ceil(H / R) blocks of 8 waves walking the slots, then a
// fixed-order sum of partial * top_w and the optional fp16 residual add.
// Lane l reads bytes [1024 j + 16 l, +16) of chunk j of a packed row (32
// codes; rows shorter than 1 KB, such as down's 512 bytes at ffn 1024: bytes
// [512 j + 8 l, +8), 16 codes) and the matching activations; codes become exact fp16 values
// (nibble masks, byte permutes against 0x64, one packed subtract) dotted with
// v_dot2_f32_f16.
#include "qformat.h"

namespace {

using namespace lemoq_qf;

// One packed row tile of R rows: KCH slices of SB bytes per row (SB = 16:
// lane l reads bytes [1024 j + 16 l, +16), 32 codes; SB = 8, for rows shorter
// than 1 KB: bytes [512 j + 8 l, +8), 16 codes, so all 64 lanes load) and
// their scales.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int SB>
struct Slice;
template <>
struct Slice<16> {
  u32x4 v;
};
template <>
struct Slice<8> {
  u32x2 v;
};

template <int R, int KCH, int SB>
struct Q4Tile {
  Slice<SB> c[R][KCH];
  uint16_t s[R][KCH];
  uint32_t ok;
};

template <int R, int KCH, int SB>
__device__ __forceinline__ void q4_issue(Q4Tile<R, KCH, SB>& t, const uint8_t* __restrict__ codes,
                                         const uint16_t* __restrict__ scale, int64_t row0, int64_t nrows,
                                         int row_bytes, int ngroups, int group, int lane) {
  t.ok = 0u;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = row0 + r;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int off = 64 * SB * j + SB * lane;
      const bool in = row < nrows && off < row_bytes;
      const int64_t rr = in ? row : 0;
      const int oo = in ? off : 0;
      const uint8_t* p = codes + rr * row_bytes + oo;
      if constexpr (SB == 16)
        t.c[r][j].v = load_stream16(reinterpret_cast<const int8_t*>(p));
      else
        t.c[r][j].v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
      t.s[r][j] = scale[rr * ngroups + (oo * 2) / group];
      t.ok |= (in ? 1u : 0u) << (r * KCH + j);
    }
  }
}

template <int KCH, int SB>
struct X4 {
  XChunk a[KCH], b[KCH];  // activations of the slice: [0, 16) and (SB = 16) [16, 32)
};

template <int KCH, int SB>
__device__ __forceinline__ void x4_load(uint32_t (&w)[KCH][SB], const uint16_t* __restrict__ x, int n, int lane) {
  const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) && ((n & 7) == 0);
#pragma unroll
  for (int j = 0; j < KCH; ++j) xq_load<2 * SB>(w[j], x, n, 128 * SB * j + 2 * SB * lane, vec);
}

template <int KCH, int SB>
__device__ __forceinline__ void x4_chunks(const uint32_t (&w)[KCH][SB], X4<KCH, SB>& x) {
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    xchunk_of(&w[j][0], x.a[j]);
    if constexpr (SB == 16) xchunk_of(&w[j][8], x.b[j]);
  }
}

// 16 packed int4 codes (two dwords) x 16 activations: dword d holds codes
// 8d .. 8d+7, the layout dot32_i4 reads from each of its four dwords.
__device__ __forceinline__ float dot16_i4(const u32x2 c, const XChunk& x, float acc) {
  const uint32_t cw[2] = {c.x, c.y};
  const f16x2 bias = {(f16)1032.0f, (f16)1032.0f};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t t = cw[d] ^ 0x88888888u;
    const uint32_t lo = t & 0x0F0F0F0Fu, hi = (t >> 4) & 0x0F0F0F0Fu;
    const int i0 = 2 * d;
    const f16x2 p0 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u)) - bias;
    const f16x2 p1 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u)) - bias;
    const f16x2 p2 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u)) - bias;
    const f16x2 p3 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)) - bias;
    acc = __builtin_amdgcn_fdot2(p0, x.a[i0], acc, false);
    acc = __builtin_amdgcn_fdot2(p1, x.a[i0 + 1], acc, false);
    acc = __builtin_amdgcn_fdot2(p2, x.b[i0], acc, false);
    acc = __builtin_amdgcn_fdot2(p3, x.b[i0 + 1], acc, false);
  }
  return acc;
}

template <int R, int KCH, int SB>
__device__ __forceinline__ float q4_row_dot(const Q4Tile<R, KCH, SB>& t, int r, const X4<KCH, SB>& x) {
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < KCH; ++j) {
    const float sc = ((t.ok >> (r * KCH + j)) & 1u) ? h2f(t.s[r][j]) : 0.0f;
    float d;
    if constexpr (SB == 16) d = dot32_i4<true>(t.c[r][j].v, x.a[j], x.b[j], 0.0f);
    else d = dot16_i4(t.c[r][j].v, x.a[j], 0.0f);
    a = fmaf(sc, d, a);
  }
  return a;
}

struct Q4GateUpArgs {
  const uint16_t* x;
  const uint8_t* codes;
  const uint16_t* scale;
  const int64_t* ids;      // plain form
  const uint16_t* logits;  // routed form: (E) fp16 router logits
  int top_k;
  int norm;
  int64_t* ids_out;        // routed form: selected ids (top_k)
  uint16_t* w_out;         // routed form: fp16 routing weights (top_k)
  int E, F, H, group;
  uint16_t* act;
};

// PL = 0: ids given; PL > 0: routed from E <= 64 * PL logits, as the 8-bit
// routed kernel (moe.hip): wave 0 of every block runs the softmax and the
// argmax rounds up to its slot's rank (wave_route), block (0, 0) runs all
// top_k rounds and stores the ids and fp16 weights for the down kernel.
template <int KCH, int R, int SB, int PL>
__global__ __launch_bounds__(256) void moe_gate_up_q4_kernel(const Q4GateUpArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = blockIdx.y;
  const uint16_t* __restrict__ x = a.x;
  const uint8_t* __restrict__ codes = a.codes;
  const uint16_t* __restrict__ scale = a.scale;
  const int E = a.E, F = a.F, H = a.H, group = a.group;
  uint16_t* __restrict__ act = a.act;
  int64_t e = 0;
  constexpr int PZ = PL > 0 ? PL : 1;
  float z[PZ];
  if constexpr (PL > 0) {
    // Unconditional loads (index clamped, value masked after the load).
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int idx = lane + 64 * i;
      const float v = h2f(a.logits[idx < E ? idx : E - 1]);
      z[i] = idx < E ? v : -INFINITY;
    }
  } else {
    e = a.ids[slot];
  }
  uint32_t xw[KCH][SB];
  x4_load<KCH, SB>(xw, x, H, lane);
  if constexpr (PL > 0) {
    __shared__ int sel_id[64];
    if (wave == 0) {
      const bool publish = blockIdx.x == 0 && slot == 0;
      const int rounds = publish ? a.top_k : slot + 1;
      int id;
      float w;
      wave_route<PZ>(z, E, a.top_k, a.norm != 0, id, w, rounds);
      if (lane < rounds) {
        sel_id[lane] = id;
        if (publish) {
          a.ids_out[lane] = (int64_t)id;
          a.w_out[lane] = f2h(w);
        }
      }
    }
    __syncthreads();
    e = sel_id[slot];
  }
  const bool ev = e >= 0 && e < E;
  const int n0 = (blockIdx.x * 4 + wave) * R;
  const int ng = H / group;
  const int rb = H / 2;
  const int64_t ebase = (ev ? e : 0) * (int64_t)(2 * F);
  const int64_t nrows = ev ? (int64_t)F : 0;  // an invalid expert id yields a zero row
  Q4Tile<R, KCH, SB> tg, tu;
  q4_issue<R, KCH, SB>(tg, codes + ebase * rb, scale + ebase * ng, n0, nrows, rb, ng, group, lane);
  q4_issue<R, KCH, SB>(tu, codes + (ebase + F) * rb, scale + (ebase + F) * ng, n0, nrows, rb, ng, group, lane);
  LEMOQ_LOADS_ISSUED();
  X4<KCH, SB> xc;
  x4_chunks<KCH, SB>(xw, xc);
  float g[R], u[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    g[r] = wave_sum(q4_row_dot<R, KCH, SB>(tg, r, xc));
    u[r] = wave_sum(q4_row_dot<R, KCH, SB>(tu, r, xc));
  }
  if (lane < R) {
    float gv = g[0], uv = u[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) {
        gv = g[r];
        uv = u[r];
      }
    if (!ev) gv = uv = 0.0f;
    const int n = n0 + lane;
    if (n < F) {
      const float sig = 1.0f / (1.0f + expf(-gv));
      act[(int64_t)slot * F + n] = f2h(gv * sig * uv);
    }
  }
}

template <int KCH, int R, int SB>
__global__ __launch_bounds__(512) void moe_down_q4_kernel(
    const uint16_t* __restrict__ act, const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scale,
    const int64_t* __restrict__ ids, const uint16_t* __restrict__ top_w, int top_k, int E, int H, int F,
    int group, const uint16_t* __restrict__ resid, uint16_t* __restrict__ out) {
  __shared__ float part[64][R];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * R;
  const int ng = F / group;
  const int rb = F / 2;
  const int t = threadIdx.x;
  const int nres = n0 + (t & (R - 1));
  const uint16_t res = *(resid ? resid + (nres < H ? nres : H - 1) : act);
  for (int slot = wave; slot < top_k; slot += 8) {
    const int64_t e = ids[slot];
    const float wslot = h2f(top_w[slot]);
    uint32_t aw[KCH][SB];
    x4_load<KCH, SB>(aw, act + (int64_t)slot * F, F, lane);
    const bool ev = e >= 0 && e < E;
    const int64_t ebase = (ev ? e : 0) * (int64_t)H;
    Q4Tile<R, KCH, SB> tl;
    q4_issue<R, KCH, SB>(tl, codes + ebase * rb, scale + ebase * ng, n0, ev ? (int64_t)H : 0, rb, ng, group,
                         lane);
    LEMOQ_LOADS_ISSUED();
    X4<KCH, SB> xc;
    x4_chunks<KCH, SB>(aw, xc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(q4_row_dot<R, KCH, SB>(tl, r, xc));
      if (lane == 0) part[slot][r] = ev ? v * wslot : 0.0f;
    }
  }
  __syncthreads();
  if (t < R) {
    const int n = n0 + t;
    if (n < H) {
      float v = 0.0f;
      for (int i = 0; i < top_k; ++i) v += part[i][t];
      uint16_t o = f2h(v);
      if (resid) o = hadd_round(h2f(o), res);
      out[n] = o;
    }
  }
}

// Slice bytes and 1 KB (SB = 16) or 512 B (SB = 8) chunks of a packed row of
// k 4-bit codes: rows shorter than 1 KB take 8-byte slices so every lane loads.
struct Q4Geom {
  int sb, kch;
};
Q4Geom q4_geom(int64_t k) {
  const int64_t rb = k / 2;
  if (rb < 1024) return {8, 1};
  const int64_t c = (rb + 1023) / 1024;
  return {16, c <= 1 ? 1 : (c <= 2 ? 2 : 4)};
}

}  // namespace

namespace {

int check_gate_up_q4(const uint16_t* x, const uint8_t* codes, const uint16_t* scale, const void* sel,
                     const uint16_t* act, int64_t top_k, int64_t num_experts, int64_t ffn, int64_t hidden,
                     int64_t group) {
  if (!x || !codes || !scale || !sel || !act) return LEMOQ_ERR_NULL;
  if (top_k <= 0 || top_k > 65535 || num_experts <= 0 || ffn <= 0 || hidden <= 0) return LEMOQ_ERR_SHAPE;
  if (hidden > 8192 || hidden % 32 != 0 || group <= 0 || group % 32 != 0 || hidden % group != 0)
    return LEMOQ_ERR_UNSUPPORTED;
  if (num_experts * 2 * ffn * hidden >= (int64_t)1 << 40) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes)) return LEMOQ_ERR_ALIGN;
  return LEMOQ_OK;
}

#ifndef LEMOQ_GUQ4_ROWS
#define LEMOQ_GUQ4_ROWS 4  // gate and up rows per wave (2: 0.498, 4: 0.490, 8: 0.509 ms per 4-bit step)
#endif

template <int PL>
int launch_gate_up_q4(hipStream_t st, const Q4GateUpArgs& a) {
  constexpr int R = LEMOQ_GUQ4_ROWS;
  const dim3 grid((unsigned)((a.F + 4 * R - 1) / (4 * R)), (unsigned)a.top_k);
  const Q4Geom geo = q4_geom(a.H);
#define LEMOQ_GU4(KK, SS) hipLaunchKernelGGL((moe_gate_up_q4_kernel<KK, R, SS, PL>), grid, dim3(256), 0, st, a)
  if (geo.sb == 8) LEMOQ_GU4(1, 8);
  else if (geo.kch == 1) LEMOQ_GU4(1, 16);
  else if (geo.kch == 2) LEMOQ_GU4(2, 16);
  else LEMOQ_GU4(4, 16);
#undef LEMOQ_GU4
  LEMOQ_CHECK_LAUNCH();
}

Q4GateUpArgs make_gate_up_q4(const uint16_t* x, const uint8_t* codes, const uint16_t* scale, int64_t top_k,
                             int64_t E, int64_t F, int64_t H, int64_t group, uint16_t* act) {
  Q4GateUpArgs a;
  a.x = x;
  a.codes = codes;
  a.scale = scale;
  a.ids = nullptr;
  a.logits = nullptr;
  a.top_k = (int)top_k;
  a.norm = 0;
  a.ids_out = nullptr;
  a.w_out = nullptr;
  a.E = (int)E;
  a.F = (int)F;
  a.H = (int)H;
  a.group = (int)group;
  a.act = act;
  return a;
}

}  // namespace

extern "C" int lemoq_moe_gate_up_w4(const uint16_t* x, const uint8_t* codes, const uint16_t* scale,
                                    const int64_t* ids, int64_t top_k, int64_t num_experts, int64_t ffn,
                                    int64_t hidden, int64_t group, uint16_t* act, void* stream) {
  const int rc = check_gate_up_q4(x, codes, scale, ids, act, top_k, num_experts, ffn, hidden, group);
  if (rc) return rc;
  Q4GateUpArgs a = make_gate_up_q4(x, codes, scale, top_k, num_experts, ffn, hidden, group, act);
  a.ids = ids;
  return launch_gate_up_q4<0>(lemoq_stream(stream), a);
}

extern "C" int lemoq_moe_gate_up_w4_routed(const uint16_t* x, const uint8_t* codes, const uint16_t* scale,
                                           const uint16_t* router_logits, int64_t top_k, int norm_topk_prob,
                                           int64_t num_experts, int64_t ffn, int64_t hidden, int64_t group,
                                           uint16_t* act, int64_t* top_i, uint16_t* top_w, void* stream) {
  const int rc = check_gate_up_q4(x, codes, scale, router_logits, act, top_k, num_experts, ffn, hidden, group);
  if (rc) return rc;
  if (!top_i || !top_w) return LEMOQ_ERR_NULL;
  if (top_k > 64 || top_k > num_experts) return LEMOQ_ERR_SHAPE;
  if (num_experts > 256) return LEMOQ_ERR_UNSUPPORTED;
  Q4GateUpArgs a = make_gate_up_q4(x, codes, scale, top_k, num_experts, ffn, hidden, group, act);
  a.logits = router_logits;
  a.norm = norm_topk_prob ? 1 : 0;
  a.ids_out = top_i;
  a.w_out = top_w;
  hipStream_t st = lemoq_stream(stream);
  return num_experts <= 64 ? launch_gate_up_q4<1>(st, a) : launch_gate_up_q4<4>(st, a);
}

extern "C" int lemoq_moe_down_w4(const uint16_t* act, const uint8_t* codes, const uint16_t* scale,
                                 const int64_t* ids, const uint16_t* top_w, int64_t top_k, int64_t num_experts,
                                 int64_t hidden, int64_t ffn, int64_t group, const uint16_t* residual,
                                 uint16_t* out, void* stream) {
  if (!act || !codes || !scale || !ids || !top_w || !out) return LEMOQ_ERR_NULL;
  if (top_k <= 0 || top_k > 64 || num_experts <= 0 || ffn <= 0 || hidden <= 0) return LEMOQ_ERR_SHAPE;
  if (ffn > 8192 || ffn % 32 != 0 || group <= 0 || group % 32 != 0 || ffn % group != 0)
    return LEMOQ_ERR_UNSUPPORTED;
  if (num_experts * hidden * ffn >= (int64_t)1 << 40) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes)) return LEMOQ_ERR_ALIGN;
#ifndef LEMOQ_DNQ4_ROWS
#define LEMOQ_DNQ4_ROWS 4  // output rows per block (2: 0.511, 4: 0.490, 8: 0.492 ms per 4-bit step)
#endif
  constexpr int R = LEMOQ_DNQ4_ROWS;
  const dim3 grid((unsigned)((hidden + R - 1) / R));
  hipStream_t st = lemoq_stream(stream);
  const int K = (int)top_k, E = (int)num_experts, H = (int)hidden, F = (int)ffn, g = (int)group;
  const Q4Geom geo = q4_geom(ffn);
#define LEMOQ_DN4(KK, SS)                                                                                 \
  hipLaunchKernelGGL((moe_down_q4_kernel<KK, R, SS>), grid, dim3(512), 0, st, act, codes, scale, ids, top_w, K, \
                     E, H, F, g, residual, out)
  if (geo.sb == 8) LEMOQ_DN4(1, 8);
  else if (geo.kch == 1) LEMOQ_DN4(1, 16);
  else if (geo.kch == 2) LEMOQ_DN4(2, 16);
  else LEMOQ_DN4(4, 16);
#undef LEMOQ_DN4
  LEMOQ_CHECK_LAUNCH();
}
