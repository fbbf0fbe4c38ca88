// Grouped MoE w8a16 GEMVs for one token: top_k of E experts, int8 codes with
// per-group fp16 scales dequantised in registers, fp32 accumulation.
//
// gate/up:  grid (ceil(F / (4*R)), top_k); wave w of block b computes the R
//           gate rows and the R matching up rows n = (4b + w)*R + r of expert
//           ids[slot] and writes act[slot, n] = fp16(silu(g) * u).  The
//           routed form takes the router's fp16 logits instead of ids: wave 0
//           of every block runs the softmax of the logits and as many argmax
//           rounds as its slot needs (wave_route: DPP max, ballot, readlane)
//           and the block streams the expert of its slot; block (0, 0) runs
//           all top_k rounds and stores the selected ids and fp16 weights for
//           the down kernel.
// down:     grid ceil(H / R) blocks of 8 waves; wave w walks the slots
//           w, w+8, ... and computes the R rows of expert ids[slot] against
//           act[slot]; the block then sums slot partials * top_w in a fixed
//           slot order (deterministic, no atomics) and applies the optional
//           fp16 residual add.
// Every wave issues all of its weight loads (plus the activation slice)
// before any arithmetic, with the lane layout of the dense GEMV (gemv.hip).
#include "common.h"

namespace {

struct GateUpArgs {
  const uint16_t* x;
  const int8_t* codes;
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

// PL = 0: ids given; PL > 0: routed from E <= 64*PL logits.
template <int KCH, int R, int PL, bool EXACT>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(const GateUpArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = blockIdx.y;
  int64_t e = 0;
  constexpr int PZ = PL > 0 ? PL : 1;
  float z[PZ];
  if constexpr (PL > 0) {
    // Unconditional loads (index clamped, value masked after the load): a
    // load under a branch is waited on before the x loads below are issued.
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int idx = lane + 64 * i;
      const float v = h2f(a.logits[idx < a.E ? idx : a.E - 1]);
      z[i] = idx < a.E ? v : -INFINITY;
    }
  } else {
    e = a.ids[slot];
  }
  XRaw<KCH> xv;
  x_issue<KCH, EXACT>(xv, a.x, a.H, true, lane);
  if constexpr (PL > 0) {
    // Routing once per block: wave 0 ranks the logits, the block reads its id
    // from LDS (the other waves' x loads are in flight meanwhile).
    __shared__ int sel_id[64];
    if (wave == 0) {
      // Block (0, 0) selects all top_k (ids and weights for the down
      // kernel); every other block stops at its own slot's rank.
      const bool publish = blockIdx.x == 0 && slot == 0;
      const int rounds = publish ? a.top_k : slot + 1;
      int id;
      float w;
      wave_route<PZ>(z, a.E, a.top_k, a.norm != 0, id, w, rounds);
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
  const bool ev = e >= 0 && e < a.E;
  const int F = a.F;
  const int n0 = (blockIdx.x * 4 + wave) * R;
  const int ng = a.H / a.group;
  const int64_t ebase = (ev ? e : 0) * (int64_t)(2 * F);
  const int64_t nrows = ev ? (int64_t)F : 0;  // an invalid expert id yields a zero row
  W8Tile<R, KCH> tg, tu;
  w8_issue<R, KCH, EXACT>(tg, a.codes + ebase * a.H, a.scale + ebase * ng, n0, nrows, a.H, ng,
                          a.group, lane);
  w8_issue<R, KCH, EXACT>(tu, a.codes + (ebase + F) * a.H, a.scale + (ebase + F) * ng, n0, nrows,
                          a.H, ng, a.group, lane);
  LEMOQ_LOADS_ISSUED();
  XChunk xc[KCH];
  x_chunks<KCH>(xv, xc);
  float g[R], u[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    g[r] = wave_sum(w8_row_dot<R, KCH>(tg, r, xc));
    u[r] = wave_sum(w8_row_dot<R, KCH>(tu, r, xc));
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
      a.act[(int64_t)slot * F + n] = f2h(gv * sig * uv);
    }
  }
}

template <int KCH, int R, bool EXACT>
__global__ __launch_bounds__(512) void moe_down_kernel(
    const uint16_t* __restrict__ act, const int8_t* __restrict__ codes,
    const uint16_t* __restrict__ scale, const int64_t* __restrict__ ids,
    const uint16_t* __restrict__ top_w, int top_k, int E, int H, int F, int group,
    const uint16_t* __restrict__ resid, uint16_t* __restrict__ out) {
  __shared__ float part[64][R];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * R;
  const int ng = F / group;
  // Epilogue operands (residual of this block's rows) are loaded up front,
  // unconditionally (a load under a branch is waited on right away).
  const int t = threadIdx.x;
  const int nres = n0 + (t & (R - 1));
  const uint16_t res = *(resid ? resid + (nres < H ? nres : H - 1) : act);

  for (int slot = wave; slot < top_k; slot += 8) {
    const int64_t e = ids[slot];
    const float wslot = h2f(top_w[slot]);
    XRaw<KCH> av;
    x_issue<KCH, EXACT>(av, act + (int64_t)slot * F, F, true, lane);
    const bool ev = e >= 0 && e < E;
    const int64_t ebase = (ev ? e : 0) * (int64_t)H;
    W8Tile<R, KCH> t;
    w8_issue<R, KCH, EXACT>(t, codes + ebase * F, scale + ebase * ng, n0, ev ? (int64_t)H : 0, F,
                            ng, group, lane);
    LEMOQ_LOADS_ISSUED();
    XChunk xc[KCH];
    x_chunks<KCH>(av, xc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(w8_row_dot<R, KCH>(t, r, xc));
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

template <int KCH>
int launch_gate_up(hipStream_t st, const GateUpArgs& a, int pl) {
  constexpr int R = 2;
  dim3 grid((unsigned)((a.F + 4 * R - 1) / (4 * R)), (unsigned)a.top_k);
  const bool exact = a.H == 1024 * KCH && a.F % (4 * R) == 0;
#define LEMOQ_GU_CASE(PP)                                                                      \
  case PP:                                                                                     \
    if (exact)                                                                                 \
      hipLaunchKernelGGL((moe_gate_up_kernel<KCH, R, PP, true>), grid, dim3(256), 0, st, a);  \
    else                                                                                       \
      hipLaunchKernelGGL((moe_gate_up_kernel<KCH, R, PP, false>), grid, dim3(256), 0, st, a); \
    break;
  switch (pl) {
    LEMOQ_GU_CASE(0)
    LEMOQ_GU_CASE(1)
    LEMOQ_GU_CASE(4)
    default: return LEMOQ_ERR_UNSUPPORTED;
  }
#undef LEMOQ_GU_CASE
  LEMOQ_CHECK_LAUNCH();
}

template <int KCH>
int launch_down(hipStream_t st, const uint16_t* act, const int8_t* codes, const uint16_t* scale,
                const int64_t* ids, const uint16_t* top_w, int top_k, int E, int H, int F,
                int group, const uint16_t* resid, uint16_t* out) {
  constexpr int R = 4;
  dim3 grid((unsigned)((H + R - 1) / R));
  if (F == 1024 * KCH && H % R == 0)
    hipLaunchKernelGGL((moe_down_kernel<KCH, R, true>), grid, dim3(512), 0, st, act, codes, scale,
                       ids, top_w, top_k, E, H, F, group, resid, out);
  else
    hipLaunchKernelGGL((moe_down_kernel<KCH, R, false>), grid, dim3(512), 0, st, act, codes,
                       scale, ids, top_w, top_k, E, H, F, group, resid, out);
  LEMOQ_CHECK_LAUNCH();
}

int kch_of(int64_t k) {
  const int64_t c = (k + 1023) / 1024;
  return c <= 1 ? 1 : (c <= 2 ? 2 : (c <= 4 ? 4 : 8));
}

int gate_up_dispatch(hipStream_t st, const GateUpArgs& a, int pl) {
  switch (kch_of(a.H)) {
    case 1: return launch_gate_up<1>(st, a, pl);
    case 2: return launch_gate_up<2>(st, a, pl);
    case 4: return launch_gate_up<4>(st, a, pl);
    default: return launch_gate_up<8>(st, a, pl);
  }
}

int check_gate_up(const uint16_t* x, const int8_t* codes, const uint16_t* scale, const void* sel,
                  uint16_t* act, int64_t top_k, int64_t num_experts, int64_t ffn, int64_t hidden,
                  int64_t group) {
  if (!x || !codes || !scale || !sel || !act) return LEMOQ_ERR_NULL;
  if (top_k <= 0 || top_k > 65535 || num_experts <= 0 || ffn <= 0 || hidden <= 0)
    return LEMOQ_ERR_SHAPE;
  if (hidden > 8192 || hidden % 16 != 0 || group <= 0 || group % 16 != 0 || hidden % group != 0)
    return LEMOQ_ERR_UNSUPPORTED;
  if (num_experts * 2 * ffn * hidden >= (int64_t)1 << 40) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes) || !lemoq_aligned16(x)) return LEMOQ_ERR_ALIGN;
  return LEMOQ_OK;
}

GateUpArgs make_gate_up(const uint16_t* x, const int8_t* codes, const uint16_t* scale,
                        int64_t top_k, int64_t E, int64_t F, int64_t H, int64_t group,
                        uint16_t* act) {
  GateUpArgs a;
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

extern "C" int lemoq_moe_gate_up_w8(const uint16_t* x, const int8_t* codes, const uint16_t* scale,
                                    const int64_t* ids, int64_t top_k, int64_t num_experts,
                                    int64_t ffn, int64_t hidden, int64_t group, uint16_t* act,
                                    void* stream) {
  int rc = check_gate_up(x, codes, scale, ids, act, top_k, num_experts, ffn, hidden, group);
  if (rc) return rc;
  GateUpArgs a = make_gate_up(x, codes, scale, top_k, num_experts, ffn, hidden, group, act);
  a.ids = ids;
  return gate_up_dispatch(lemoq_stream(stream), a, 0);
}

extern "C" int lemoq_moe_gate_up_w8_routed(const uint16_t* x, const int8_t* codes,
                                           const uint16_t* scale, const uint16_t* router_logits,
                                           int64_t top_k, int norm_topk_prob,
                                           int64_t num_experts, int64_t ffn, int64_t hidden,
                                           int64_t group, uint16_t* act, int64_t* top_i,
                                           uint16_t* top_w, void* stream) {
  int rc = check_gate_up(x, codes, scale, router_logits, act, top_k, num_experts, ffn, hidden,
                         group);
  if (rc) return rc;
  if (!top_i || !top_w) return LEMOQ_ERR_NULL;
  if (top_k > 64 || top_k > num_experts) return LEMOQ_ERR_SHAPE;
  if (num_experts > 256) return LEMOQ_ERR_UNSUPPORTED;
  GateUpArgs a = make_gate_up(x, codes, scale, top_k, num_experts, ffn, hidden, group, act);
  a.logits = router_logits;
  a.norm = norm_topk_prob ? 1 : 0;
  a.ids_out = top_i;
  a.w_out = top_w;
  return gate_up_dispatch(lemoq_stream(stream), a, num_experts <= 64 ? 1 : 4);
}

extern "C" int lemoq_moe_down_w8(const uint16_t* act, const int8_t* codes, const uint16_t* scale,
                                 const int64_t* ids, const uint16_t* top_w, int64_t top_k,
                                 int64_t num_experts, int64_t hidden, int64_t ffn, int64_t group,
                                 const uint16_t* residual, uint16_t* out, void* stream) {
  if (!act || !codes || !scale || !ids || !top_w || !out) return LEMOQ_ERR_NULL;
  if (top_k <= 0 || top_k > 64 || num_experts <= 0 || ffn <= 0 || hidden <= 0)
    return LEMOQ_ERR_SHAPE;
  if (ffn > 8192 || ffn % 16 != 0 || group <= 0 || group % 16 != 0 || ffn % group != 0)
    return LEMOQ_ERR_UNSUPPORTED;
  if (num_experts * hidden * ffn >= (int64_t)1 << 40) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes) || !lemoq_aligned16(act)) return LEMOQ_ERR_ALIGN;
  hipStream_t st = lemoq_stream(stream);
  switch (kch_of(ffn)) {
    case 1: return launch_down<1>(st, act, codes, scale, ids, top_w, (int)top_k, (int)num_experts, (int)hidden, (int)ffn, (int)group, residual, out);
    case 2: return launch_down<2>(st, act, codes, scale, ids, top_w, (int)top_k, (int)num_experts, (int)hidden, (int)ffn, (int)group, residual, out);
    case 4: return launch_down<4>(st, act, codes, scale, ids, top_w, (int)top_k, (int)num_experts, (int)hidden, (int)ffn, (int)group, residual, out);
    default: return launch_down<8>(st, act, codes, scale, ids, top_w, (int)top_k, (int)num_experts, (int)hidden, (int)ffn, (int)group, residual, out);
  }
}
