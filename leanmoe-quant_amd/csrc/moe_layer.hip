// The grouped MoE of one decoder layer at batch 1 as ONE launch: routing,
// gate/up + SiLU and down x routing weight + residual -- the work of
// moe_gate_up_w8_routed followed by moe_down_w8, with their arithmetic (every
// output is bit-identical to theirs).
//
// What the fusion buys: the selected experts' down weights stream in during
// the gate/up phase (their addresses are known once the block has routed), so
// the down projection no longer pays a launch, a dependent id load and its
// own first-load latency.
//
// Grid: top_k * B workgroups of 8 waves, all resident at once (the entry
// point checks the kernel's occupancy); workgroup b serves slot s = b / B and
// part j = b % B of it.  Every workgroup routes the token itself (softmax and
// top_k argmax rounds of the fp16 logits, ties -> lowest index), then
//   1  issues its gate/up rows (F / (8 B) rows per wave) and its down rows
//      (H / (8 B) rows per wave) of expert ids[s], computes
//      act = fp16(silu(g) * u) for its gate/up rows, stores them coherently
//      and counts itself in on slot s's counter;
//   2  waits for the B workgroups of slot s, reads act[s] and computes its
//      down rows x the slot's fp16 routing weight (fp32 partials, stored
//      coherently), counting itself in on its row range's counter;
//   3  waits for the top_k workgroups (one per slot) that computed its H / G
//      output rows, sums the slots' partials in slot order, rounds to fp16
//      and adds the residual.
// Hand-offs use sync.h: coherent stores, counters, bounded waits.  The last
// workgroup through each wait returns that wait's counters to zero.
#include "sync.h"

namespace {

constexpr int kWaves = 8;
constexpr int kMaxSlots = 16;     // top_k
constexpr int kMaxParts = 64;     // B
constexpr int kLineBase = 64;     // first sync line (lines 1..63 belong to attn_layer)

struct MoeLayerArgs {
  const uint16_t* x;       // (H) normed input
  const uint16_t* logits;  // (E) fp16 router logits
  const int8_t* gu_codes;  // (E, 2F, H)
  const uint16_t* gu_scale;
  const int8_t* dn_codes;  // (E, H, F)
  const uint16_t* dn_scale;
  int top_k, norm, E, F, H, group, parts;
  uint16_t* act;           // (top_k, F) fp16, coherent hand-off
  float* ypart;            // (top_k, H) fp32, coherent hand-off
  const uint16_t* resid;   // (H)
  uint16_t* out;           // (H)
  int64_t* ids_out;        // (top_k), written by workgroup 0
  uint16_t* w_out;         // (top_k) fp16
  uint32_t* sync;
  uint64_t limit_ticks;
};

__device__ __forceinline__ uint32_t* mline(const MoeLayerArgs& a, int i) {
  return a.sync + (int64_t)(kLineBase + i) * lemoq_sync::kLineWords;
}

__device__ __forceinline__ bool block_ok(bool wave0_ok, int* s_flag) {
  if (threadIdx.x == 0) *s_flag = wave0_ok ? 1 : 0;
  __syncthreads();
  const bool ok = *s_flag != 0;
  __syncthreads();
  return ok;
}

__device__ __forceinline__ void publish(uint32_t* counter) {
  lemoq_sync::wait_own_stores();
  __syncthreads();
  if (threadIdx.x == 0) lemoq_sync::arrive(counter);
}

// After a wait: count this workgroup through; the last of `n` returns the
// waited-on counter and this one to zero (nobody reads them any more).
__device__ __forceinline__ void passed(uint32_t* waited, uint32_t* through, uint32_t n) {
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(through, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == n - 1) {
      lemoq_sync::st_u32(waited, 0u);
      lemoq_sync::st_u32(through, 0u);
    }
  }
}

// KG = H / 1024, RG gate/up rows per wave, KD = F / 1024, RD down rows per
// wave, PL: E <= 64 * PL logits.
template <int KG, int RG, int KD, int RD, int PL>
__global__ __launch_bounds__(64 * kWaves) void moe_layer_kernel(const MoeLayerArgs a) {
  __shared__ int sel_id[kMaxSlots];
  __shared__ float sel_w[kMaxSlots];
  __shared__ int s_flag;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = gridDim.x, b = blockIdx.x;
  const int B = a.parts, s = b / B, j = b % B;
  const int F = a.F, H = a.H;
  const int CR = H / G;                   // output rows summed by this workgroup
  const int c0 = b * CR;
  uint32_t* status = a.sync;

  // Loads that need no routing: the logits (wave 0), x, the residual of the
  // rows this workgroup finishes.
  float z[PL];
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int idx = lane + 64 * i;
      const float v = h2f(a.logits[idx < a.E ? idx : a.E - 1]);
      z[i] = idx < a.E ? v : -INFINITY;
    }
  }
  XRaw<KG> xv;
  x_issue<KG, true>(xv, a.x, H, true, lane);
  const uint16_t res = a.resid[c0 + (threadIdx.x < CR ? threadIdx.x : 0)];
  if (wave == 0) {
    int id;
    float w;
    wave_route<PL>(z, a.E, a.top_k, a.norm != 0, id, w, a.top_k);
    if (lane < a.top_k) {
      const uint16_t w16 = f2h(w);
      sel_id[lane] = id;
      sel_w[lane] = h2f(w16);  // the down projection uses the fp16 routing weight
      if (b == 0) {
        a.ids_out[lane] = (int64_t)id;
        a.w_out[lane] = w16;
      }
    }
  }
  __syncthreads();
  const int64_t e = sel_id[s];
  const float ws = sel_w[s];
  const bool ev = e >= 0 && e < a.E;
  const int64_t ee = ev ? e : 0;

  // 1. gate/up rows n0 .. n0 + RG of expert e, and (loaded now, used in 2) the
  //    down rows r0 .. r0 + RD.
  const int n0 = (j * kWaves + wave) * RG;
  const int r0 = (j * kWaves + wave) * RD;
  const int ngu = H / a.group, ndn = F / a.group;
  const int64_t gbase = ee * (int64_t)(2 * F);
  W8Tile<RG, KG> tg, tu;
  w8_issue<RG, KG, true>(tg, a.gu_codes + gbase * H, a.gu_scale + gbase * ngu, n0, F, H, ngu, a.group, lane);
  w8_issue<RG, KG, true>(tu, a.gu_codes + (gbase + F) * H, a.gu_scale + (gbase + F) * ngu, n0, F, H, ngu,
                         a.group, lane);
  W8Tile<RD, KD> td;
  const int64_t dbase = ee * (int64_t)H;
  w8_issue<RD, KD, true>(td, a.dn_codes + dbase * F, a.dn_scale + dbase * ndn, r0, H, F, ndn, a.group, lane);
  LEMOQ_LOADS_ISSUED();
  {
    XChunk xc[KG];
    x_chunks<KG>(xv, xc);
    float g[RG], u[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      g[r] = wave_sum(w8_row_dot<RG, KG>(tg, r, xc));
      u[r] = wave_sum(w8_row_dot<RG, KG>(tu, r, xc));
    }
    float gv = g[0], uv = u[0];
#pragma unroll
    for (int r = 1; r < RG; ++r)
      if (lane == r) {
        gv = g[r];
        uv = u[r];
      }
    if (!ev) gv = uv = 0.0f;
    const float sig = 1.0f / (1.0f + expf(-gv));
    const uint32_t av = f2h(gv * sig * uv);
    const uint32_t hi = __shfl_down(av, 1, 64);
    // lane 2i stores act rows n0 + 2i, n0 + 2i + 1 as one coherent dword
    if (lane < RG && (lane & 1) == 0)
      lemoq_sync::st_u32(reinterpret_cast<uint32_t*>(a.act + (int64_t)s * F + n0 + lane), av | (hi << 16));
  }
  publish(mline(a, s));

  // 2. down rows of slot s, once its act row is complete.
  bool ok = true;
  if (wave == 0) ok = lemoq_sync::wait_counts(mline(a, s), 1, (uint32_t)B, status, a.limit_ticks);
  if (!block_ok(ok, &s_flag)) return;
  passed(mline(a, s), mline(a, a.top_k + s), (uint32_t)B);
  {
    XRaw<KD> avx;
#pragma unroll
    for (int jj = 0; jj < KD; ++jj) {
      const uint16_t* src = a.act + (int64_t)s * F + 1024 * jj + 16 * lane;
      avx.v[jj][0] = lemoq_sync::ld_16(src);
      avx.v[jj][1] = lemoq_sync::ld_16(src + 8);
    }
    XChunk xc[KD];
    x_chunks<KD>(avx, xc);
    float pv = 0.0f;
#pragma unroll
    for (int r = 0; r < RD; ++r) {
      const float v = wave_sum(w8_row_dot<RD, KD>(td, r, xc));
      if (lane == r) pv = ev ? v * ws : 0.0f;
    }
    if (lane < RD) lemoq_sync::st_f32(a.ypart + (int64_t)s * H + r0 + lane, pv);
  }
  publish(mline(a, 2 * a.top_k + j));

  // 3. the slots' partials of rows c0 .. c0 + CR, summed in slot order.
  const int rr = c0 / (kWaves * RD);  // the down row range holding them
  const uint32_t finishers = (uint32_t)(kWaves * RD / CR);
  if (wave == 0) ok = lemoq_sync::wait_counts(mline(a, 2 * a.top_k + rr), 1, (uint32_t)a.top_k, status, a.limit_ticks);
  if (!block_ok(ok, &s_flag)) return;
  passed(mline(a, 2 * a.top_k + rr), mline(a, 2 * a.top_k + B + rr), finishers);
  if (threadIdx.x < CR) {
    const int n = c0 + threadIdx.x;
    float v = 0.0f;
    for (int i = 0; i < a.top_k; ++i) v += lemoq_sync::ld_f32(a.ypart + (int64_t)i * H + n);
    uint16_t o = f2h(v);
    o = hadd_round(h2f(o), res);
    a.out[n] = o;
  }
}

template <int KG, int RG, int KD, int RD, int PL>
int resident(int device) {
  static int cache[64];
  static bool known[64];
  if (device < 0 || device >= 64) return 0;
  if (!known[device]) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, moe_layer_kernel<KG, RG, KD, RD, PL>, 64 * kWaves,
                                                     0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return 0;
    cache[device] = per_cu * cus;
    known[device] = true;
  }
  return cache[device];
}

// The one instance this build compiles: OLMoE's H 2048, F 1024, 32
// workgroups per slot (4 gate/up and 8 down rows per wave), E <= 64.
constexpr int kParts = 32;

int shape_ok(int64_t top_k, int64_t E, int64_t F, int64_t H, int64_t group) {
  if (H != 2048 || F != 1024 || E <= 0 || E > 64 || top_k <= 0 || top_k > kMaxSlots || top_k > E)
    return LEMOQ_ERR_UNSUPPORTED;
  if (group <= 0 || group % 16 != 0 || F % group != 0 || H % group != 0) return LEMOQ_ERR_UNSUPPORTED;
  const int64_t G = top_k * kParts;
  if (H % G != 0 || (kWaves * (H / (kParts * kWaves))) % (H / G) != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (kLineBase + 2 * top_k + 2 * kParts > LEMOQ_SYNC_WORDS / lemoq_sync::kLineWords) return LEMOQ_ERR_SHAPE;
  return LEMOQ_OK;
}

}  // namespace

extern "C" int lemoq_moe_layer_check(int64_t top_k, int64_t num_experts, int64_t ffn, int64_t hidden,
                                     int64_t group) {
  const int rc = shape_ok(top_k, num_experts, ffn, hidden, group);
  if (rc) return rc;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return LEMOQ_ERR_UNSUPPORTED;
  return resident<2, 4, 1, 8, 1>(device) >= top_k * kParts ? LEMOQ_OK : LEMOQ_ERR_UNSUPPORTED;
}

extern "C" int lemoq_moe_layer_w8(const uint16_t* x, const int8_t* gu_codes, const uint16_t* gu_scale,
                                  const int8_t* dn_codes, const uint16_t* dn_scale,
                                  const uint16_t* router_logits, int64_t top_k, int norm_topk_prob,
                                  int64_t num_experts, int64_t ffn, int64_t hidden, int64_t group,
                                  uint16_t* act, float* ypart, const uint16_t* residual, uint16_t* out,
                                  int64_t* top_i, uint16_t* top_w, uint32_t* sync, int64_t timeout_us,
                                  void* stream) {
  if (!x || !gu_codes || !gu_scale || !dn_codes || !dn_scale || !router_logits || !act || !ypart ||
      !residual || !out || !top_i || !top_w || !sync)
    return LEMOQ_ERR_NULL;
  if (timeout_us < 0) return LEMOQ_ERR_SHAPE;
  const int rc = lemoq_moe_layer_check(top_k, num_experts, ffn, hidden, group);
  if (rc) return rc;
  if (!lemoq_aligned16(x) || !lemoq_aligned16(gu_codes) || !lemoq_aligned16(dn_codes) || !lemoq_aligned16(act) ||
      !lemoq_aligned16(ypart) || (reinterpret_cast<uintptr_t>(sync) & 255u) != 0)
    return LEMOQ_ERR_ALIGN;
  MoeLayerArgs a;
  a.x = x;
  a.logits = router_logits;
  a.gu_codes = gu_codes;
  a.gu_scale = gu_scale;
  a.dn_codes = dn_codes;
  a.dn_scale = dn_scale;
  a.top_k = (int)top_k;
  a.norm = norm_topk_prob ? 1 : 0;
  a.E = (int)num_experts;
  a.F = (int)ffn;
  a.H = (int)hidden;
  a.group = (int)group;
  a.parts = kParts;
  a.act = act;
  a.ypart = ypart;
  a.resid = residual;
  a.out = out;
  a.ids_out = top_i;
  a.w_out = top_w;
  a.sync = sync;
  a.limit_ticks = (uint64_t)timeout_us * 100u;  // s_memrealtime runs at 100 MHz
  const unsigned G = (unsigned)(top_k * kParts);
  hipLaunchKernelGGL((moe_layer_kernel<2, 4, 1, 8, 1>), dim3(G), dim3(64 * kWaves), 0, lemoq_stream(stream), a);
  LEMOQ_CHECK_LAUNCH();
}
