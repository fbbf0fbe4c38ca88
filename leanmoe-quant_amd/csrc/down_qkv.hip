// The MoE down projection of decoder layer L and the packed q|k|v GEMV of
// layer L+1 as ONE launch (batch 1), with the arithmetic of moe_down_w8
// followed by gemv_w8_fused (input RMSNorm prologue): every output bit is
// theirs.
//
// What the fusion buys: the q|k|v weight rows of layer L+1 (12.8 MB at the
// OLMoE shape) do not depend on anything the down projection computes, so
// every workgroup issues them at entry, next to its down rows.  When the
// residual stream h is complete, the workgroups only normalise it and dot it
// with rows already in registers: the launch boundary, the q|k|v kernel's
// first-load latency and its weight stream all leave the critical path.
//
// Grid: H / 4 workgroups of 8 waves (512 threads), all resident at once (the
// entry point checks the kernel's occupancy).  Workgroup b
//   1  loads its slot ids and routing weights, the residual of its rows
//      4b .. 4b+3, its n_qkv / (H / 4) q|k|v rows (2 per wave, the first
//      rows/2 waves) and the norm weight;
//   2  as moe_down_w8 (R = 4): wave w streams the 4 down rows of expert
//      ids[w] against act[w], the block sums the slots' partials x weight in
//      slot order, rounds to fp16 and adds the residual; stores h rows
//      4b .. 4b+3 (plain stores, for later launches) and publishes them to
//      the other workgroups;
//   3  waits until all H values are published, then runs the block RMSNorm
//      of gemv_w8_fused (threads 0..255 each sum 8 values in column order,
//      wave sums, the four wave totals in wave order) into LDS, and each wave
//      with rows dots them and stores fp16 q|k|v.
//
// The hand-off needs no counters and no wait for stores: h moves in 64-bit
// words that carry 2 fp16 values in the low half and a flag in the high half,
// written and read with relaxed agent-scope atomics (global_store/load
// dwordx2 with the sc1 scope bit, coherent across the XCDs' L2s).  A 64-bit
// store is seen whole or not at all, so a reader that sees the flag sees the
// values.  The flag is unique to the launch: 2 * gen + 1, where gen is a
// launch counter in the sync workspace that every workgroup reads at entry
// and workgroup 0 advances once its wait has passed (every workgroup has
// published by then, so every one has read it).  Words left by earlier
// launches carry other flags and are never taken for this launch's, so the
// buffer needs no clearing between launches (a first flag of 1 against a
// zeroed buffer and counter).  Every wait is bounded by a time limit
// (s_memrealtime, 100 MHz); on expiry the workgroup records
// LEMOQ_SYNC_TIMEOUT_BIT in the status word, skips its q|k|v rows and
// returns, so the grid always drains.  (The poll does not read the status
// word: every workgroup gives up on its own clock.)
#include <mutex>

#include "sync.h"

namespace {

constexpr int kDQWaves = 8;
constexpr int kDQThreads = 64 * kDQWaves;
constexpr int kDownRows = 4;  // h rows per workgroup (moe_down_w8's R)
constexpr int kQkvR = 2;      // q|k|v rows per wave (gemv_w8_fused's R)

struct DownQkvArgs {
  // down projection of layer L (moe_down_w8)
  const uint16_t* act;  // (top_k, F)
  const int8_t* dn_codes;
  const uint16_t* dn_scale;
  const int64_t* ids;
  const uint16_t* top_w;
  int top_k, E, H, F, group;
  const uint16_t* resid;  // (H)
  uint16_t* h_out;        // (H)
  // input RMSNorm + q|k|v of layer L+1 (gemv_w8_fused)
  const uint16_t* norm_w;
  float eps;
  const int8_t* qkv_codes;
  const uint16_t* qkv_scale;
  int n_qkv;
  int qkv_waves;  // waves with rows: n_qkv / (H / 4) / 2
  uint16_t* qkv_out;
  // hand-off
  uint64_t* ll;      // (H / 2) words
  uint32_t* status;  // sync[0]
  uint32_t* gen;     // sync[1]: launch counter
  uint64_t limit_ticks;
};

__device__ __forceinline__ void st_ll(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_ll(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// KD: 1 KB chunks of a down row (F / 1024); KQ: of a q|k|v row (H / 1024).
template <int KD, int KQ>
__global__ __launch_bounds__(kDQThreads) void down_qkv_kernel(const DownQkvArgs a) {
  static_assert(KQ == 2 || KQ == 4 || KQ == 8, "the block norm needs H = 2048 * NV");
  constexpr int NV = KQ / 2;  // 8-value chunks per thread of the norm (threads 0..255)
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int b = blockIdx.x;
  const int n0 = b * kDownRows;
  __shared__ float part[kDQWaves][kDownRows];
  __shared__ __align__(16) uint16_t xs[KQ * 1024];
  __shared__ float red[4];

  // 1. Loads that depend on nothing this launch computes.
  const uint32_t flag = 2u * *a.gen + 1u;
  const bool has_slot = wave < a.top_k;
  const int slot = has_slot ? wave : 0;
  const int64_t e = a.ids[slot];
  const float wslot = h2f(a.top_w[slot]);
  const uint16_t res = a.resid[n0 + (t & (kDownRows - 1))];
  // q|k|v rows: waves without rows re-read wave 0's (same workgroup, L2 hits).
  const int qw = wave < a.qkv_waves ? wave : 0;
  const int64_t qrow0 = ((int64_t)b * a.qkv_waves + qw) * kQkvR;
  W8Tile<kQkvR, KQ> tq;
  w8_issue<kQkvR, KQ, true>(tq, a.qkv_codes, a.qkv_scale, qrow0, a.n_qkv, a.H, a.H / a.group,
                            a.group, lane);
  u32x4 wv[NV];
  if (t < 256) {
#pragma unroll
    for (int i = 0; i < NV; ++i) wv[i] = *reinterpret_cast<const u32x4*>(a.norm_w + (i * 256 + t) * 8);
  }
  // Down rows of this wave's slot (the id is needed for their addresses).
  const bool ev = has_slot && e >= 0 && e < a.E;
  const int ng = a.F / a.group;
  const int64_t ebase = (ev ? e : 0) * (int64_t)a.H;
  XRaw<KD> av;
  x_issue<KD, true>(av, a.act + (int64_t)slot * a.F, a.F, true, lane);
  W8Tile<kDownRows, KD> td;
  w8_issue<kDownRows, KD, true>(td, a.dn_codes + ebase * a.F, a.dn_scale + ebase * ng, n0, a.H, a.F,
                                ng, a.group, lane);
  LEMOQ_LOADS_ISSUED();

  // 2. Down projection x routing weight, slot sum, residual.
  {
    XChunk xc[KD];
    x_chunks<KD>(av, xc);
#pragma unroll
    for (int r = 0; r < kDownRows; ++r) {
      const float v = wave_sum(w8_row_dot<kDownRows, KD>(td, r, xc));
      if (lane == 0 && has_slot) part[wave][r] = ev ? v * wslot : 0.0f;
    }
  }
  __syncthreads();
  if (wave == 0) {
    uint32_t o = 0u;
    if (lane < kDownRows) {
      float v = 0.0f;
      for (int i = 0; i < a.top_k; ++i) v += part[i][lane];
      o = hadd_round(h2f(f2h(v)), res);
      a.h_out[n0 + lane] = (uint16_t)o;
    }
    // lanes 0 and 2 pack their value with the next lane's into one word
    const uint32_t hi = (uint32_t)__shfl_down((int)o, 1, 64);
    if (lane == 0 || lane == 2) {
      const int64_t wi = (int64_t)b * (kDownRows / 2) + (lane >> 1);
      st_ll(a.ll + wi, ((uint64_t)flag << 32) | (uint64_t)(o | (hi << 16)));
    }
  }

  // 3. Wait for the whole of h: thread t < 256 needs values 8 (i*256 + t) .. +8,
  // i.e. words 4 (i*256 + t) .. +4.  One barrier per poll: each wave votes
  // (wave 0 also says whether the time limit has passed) into one of two LDS
  // slots, alternating, so a slot is rewritten only after a later barrier.
  u32x4 rv[NV];
  bool failed = false;
  {
    __shared__ int vote[2][kDQWaves];
    const uint64_t t0 = lemoq_sync::now_ticks();
    for (int it = 0;; ++it) {
      bool ok = true;
      if (t < 256) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const uint64_t* p = a.ll + (int64_t)(i * 256 + t) * 4;
          const uint64_t w0 = ld_ll(p), w1 = ld_ll(p + 1), w2 = ld_ll(p + 2), w3 = ld_ll(p + 3);
          ok = ok && (uint32_t)(w0 >> 32) == flag && (uint32_t)(w1 >> 32) == flag &&
               (uint32_t)(w2 >> 32) == flag && (uint32_t)(w3 >> 32) == flag;
          rv[i] = (u32x4){(uint32_t)w0, (uint32_t)w1, (uint32_t)w2, (uint32_t)w3};
        }
      }
      const bool late = wave == 0 && lemoq_sync::now_ticks() - t0 > a.limit_ticks;
      const int v = (__all(ok) ? 1 : 0) | (late ? 2 : 0);
      if (lane == 0) vote[it & 1][wave] = v;
      __syncthreads();
      int all = 1;
#pragma unroll
      for (int w = 0; w < kDQWaves; ++w) all &= vote[it & 1][w];
      if (all & 1) break;
      if (vote[it & 1][0] & 2) {
        if (t == 0)
          __hip_atomic_fetch_or(a.status, (uint32_t)LEMOQ_SYNC_TIMEOUT_BIT, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
        failed = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  // Every workgroup has read gen before publishing, so it can move on now.
  if (b == 0 && t == 0) *a.gen = (flag + 1u) >> 1;
  if (failed) return;  // block-uniform

  // 4. Input RMSNorm of layer L+1 (gemv_w8_fused's block prologue) into LDS.
  if (t < 256) {
    float ssq = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t q[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = h2f((uint16_t)(q[k] & 0xFFFFu)), x1 = h2f((uint16_t)(q[k] >> 16));
        ssq = fmaf(x0, x0, ssq);
        ssq = fmaf(x1, x1, ssq);
      }
    }
    ssq = wave_sum(ssq);
    if (lane == 0) red[wave] = ssq;
  }
  __syncthreads();
  if (t < 256) {
    const float rstd = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)a.H + a.eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t q[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
      const uint32_t g[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint16_t m0 = f2h(h2f((uint16_t)(q[k] & 0xFFFFu)) * rstd);
        const uint16_t m1 = f2h(h2f((uint16_t)(q[k] >> 16)) * rstd);
        const uint16_t y0 = f2h(h2f(m0) * h2f((uint16_t)(g[k] & 0xFFFFu)));
        const uint16_t y1 = f2h(h2f(m1) * h2f((uint16_t)(g[k] >> 16)));
        o[k] = (uint32_t)y0 | ((uint32_t)y1 << 16);
      }
      *reinterpret_cast<u32x4*>(xs + (i * 256 + t) * 8) = (u32x4){o[0], o[1], o[2], o[3]};
    }
  }
  __syncthreads();

  // 5. q|k|v rows of this wave.
  if (wave >= a.qkv_waves) return;
  XRaw<KQ> xv;
#pragma unroll
  for (int j = 0; j < KQ; ++j) {
    xv.v[j][0] = *reinterpret_cast<const u32x4*>(xs + 1024 * j + 16 * lane);
    xv.v[j][1] = *reinterpret_cast<const u32x4*>(xs + 1024 * j + 16 * lane + 8);
  }
  XChunk xc[KQ];
  x_chunks<KQ>(xv, xc);
  float acc[kQkvR];
#pragma unroll
  for (int r = 0; r < kQkvR; ++r) acc[r] = wave_sum(w8_row_dot<kQkvR, KQ>(tq, r, xc));
  if (lane < kQkvR) a.qkv_out[qrow0 + lane] = f2h(lane == 0 ? acc[0] : acc[1]);
}

template <int KD, int KQ>
int resident_blocks(int device) {
  // Workgroups of this instance resident at once on `device`; computed once
  // per device under a lock (0 when the query fails).
  static std::mutex mu;
  static int cache[64];
  static bool known[64];
  if (device < 0 || device >= 64) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (!known[device]) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, down_qkv_kernel<KD, KQ>, kDQThreads, 0) !=
            hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return 0;
    cache[device] = per_cu * cus;
    known[device] = true;
  }
  return cache[device];
}

}  // namespace

extern "C" int lemoq_moe_down_qkv_check(int64_t top_k, int64_t hidden, int64_t ffn, int64_t group,
                                        int64_t n_qkv) {
  if (hidden != 2048 || ffn != 1024) return LEMOQ_ERR_UNSUPPORTED;
  if (top_k <= 0 || top_k > kDQWaves) return LEMOQ_ERR_UNSUPPORTED;
  if (group <= 0 || group % 16 != 0 || ffn % group != 0 || hidden % group != 0) return LEMOQ_ERR_UNSUPPORTED;
  const int64_t G = hidden / kDownRows;
  if (n_qkv <= 0 || n_qkv % (G * kQkvR) != 0 || n_qkv / (G * kQkvR) > kDQWaves) return LEMOQ_ERR_UNSUPPORTED;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return LEMOQ_ERR_UNSUPPORTED;
  return resident_blocks<1, 2>(device) >= G ? LEMOQ_OK : LEMOQ_ERR_UNSUPPORTED;
}

extern "C" int lemoq_moe_down_qkv_w8(const uint16_t* act, const int8_t* dn_codes, const uint16_t* dn_scale,
                                     const int64_t* ids, const uint16_t* top_w, int64_t top_k,
                                     int64_t num_experts, int64_t hidden, int64_t ffn, int64_t group,
                                     const uint16_t* residual, uint16_t* h_out, const uint16_t* norm_w,
                                     float eps, const int8_t* qkv_codes, const uint16_t* qkv_scale,
                                     int64_t n_qkv, uint16_t* qkv_out, uint64_t* ll, uint32_t* sync,
                                     int64_t timeout_us, void* stream) {
  if (!act || !dn_codes || !dn_scale || !ids || !top_w || !residual || !h_out || !norm_w || !qkv_codes ||
      !qkv_scale || !qkv_out || !ll || !sync)
    return LEMOQ_ERR_NULL;
  if (timeout_us < 0 || num_experts <= 0 || num_experts * hidden * ffn >= ((int64_t)1 << 40))
    return LEMOQ_ERR_SHAPE;
  const int rc = lemoq_moe_down_qkv_check(top_k, hidden, ffn, group, n_qkv);
  if (rc) return rc;
  if (!lemoq_aligned16(act) || !lemoq_aligned16(dn_codes) || !lemoq_aligned16(norm_w) ||
      !lemoq_aligned16(qkv_codes) || (reinterpret_cast<uintptr_t>(ll) & 255u) != 0 ||
      (reinterpret_cast<uintptr_t>(sync) & 7u) != 0)
    return LEMOQ_ERR_ALIGN;
  {
    const char* l0 = reinterpret_cast<const char*>(ll);
    const char* s0 = reinterpret_cast<const char*>(sync);
    if (s0 < l0 + hidden * 4 && l0 < s0 + 8) return LEMOQ_ERR_SHAPE;  // the words must not overlap
  }
  DownQkvArgs a;
  a.act = act;
  a.dn_codes = dn_codes;
  a.dn_scale = dn_scale;
  a.ids = ids;
  a.top_w = top_w;
  a.top_k = (int)top_k;
  a.E = (int)num_experts;
  a.H = (int)hidden;
  a.F = (int)ffn;
  a.group = (int)group;
  a.resid = residual;
  a.h_out = h_out;
  a.norm_w = norm_w;
  a.eps = eps;
  a.qkv_codes = qkv_codes;
  a.qkv_scale = qkv_scale;
  a.n_qkv = (int)n_qkv;
  const int G = (int)(hidden / kDownRows);
  a.qkv_waves = (int)(n_qkv / ((int64_t)G * kQkvR));
  a.qkv_out = qkv_out;
  a.ll = ll;
  a.status = sync;
  a.gen = sync + 1;
  a.limit_ticks = (uint64_t)timeout_us * 100u;  // s_memrealtime runs at 100 MHz
  hipLaunchKernelGGL((down_qkv_kernel<1, 2>), dim3((unsigned)G), dim3(kDQThreads), 0, lemoq_stream(stream), a);
  LEMOQ_CHECK_LAUNCH();
}
