// The attention half of an OLMoE decoder layer at batch 1 as ONE launch:
// split-KV attention over the KV-INT8 cache, the LSE merge + o_proj, and the
// residual + post-attention RMSNorm + router logits -- the work of the three
// launches attn_split_fused_i8, attn_merge_o_proj_w8 and router_logits_resid,
// with the same arithmetic (every output is bit-identical to theirs).
//
// Grid: heads * num_splits workgroups of 4 waves, all resident at once (the
// entry point checks the kernel's occupancy).  Workgroup b plays three roles
// in turn; a role waits only for the workgroups whose results it reads
// (sync.h: coherent stores, a counter per producer set, bounded polling):
//   A  split block (sp, h) = (b % ns, b / ns): q/k norm, RoPE, KV-INT8 write
//      of the new token, online softmax over its cached tokens; the (m, l,
//      acc) partial goes out with coherent stores and the head's counter is
//      incremented.
//   B  o_proj tile t = b (+ G, ...): waits for the ns split blocks of each of
//      its 4 heads, merges them and dots its 32 o_proj rows with the 512
//      merged features (the tile's weight slices are loaded at kernel entry,
//      before role A); increments counter t % 16.
//   C  router block b < ceil(E / 4): waits for every o_proj tile, then
//      o = fp16(sum of the partials), h' = fp16(o + h), RMSNorm and the fp16
//      logits of its 4 experts (router rows, h and the norm weight are loaded
//      at entry); the last router block to finish returns the counters to 0.
// Two kernel boundaries per layer are gone: the o_proj and router launches'
// dispatch, first loads and tail are replaced by two waits on small
// producer sets (16 and 256 arrivals spread over 16 counters).
#include "attn_fused.h"
#include "oproj_router.h"
#include "sync.h"

namespace {

using lemoq_attn_fused::AttnSplitArgs;
using namespace lemoq_oproj;

constexpr int kTileLines = 16;  // o_proj tile counters (tile t arrives on t % 16)

// Sync workspace lines (uint32 words, 64 per line): 0 status; 1 + h: split
// blocks of head h; 1 + heads + k: o_proj tiles t with t % 16 == k; then the
// router blocks.
struct LayerArgs {
  AttnSplitArgs at;
  MergeOprojArgs mo;
  RouterResidArgs rr;
  uint32_t* sync;
  uint64_t limit_ticks;
  int n_tiles;     // o_proj tiles: (N / 32) * (heads / 4)
  int row_blocks;  // N / 32
  int n_router;    // router blocks: ceil(E / 4)
};

__device__ __forceinline__ uint32_t* line(const LayerArgs& a, int i) {
  return a.sync + (int64_t)i * lemoq_sync::kLineWords;
}

// o_proj tile t -> (head group g, row block rb).  When the group count divides
// 8 and the tiles fill whole rounds of the 8 XCDs, tiles on one XCD (t % 8)
// share a head group, so each L2 serves one group's split partials.
__device__ __forceinline__ void tile_coords(int t, int groups, int rbs, int n_tiles, int& g, int& rb) {
  if (8 % groups == 0 && n_tiles % 8 == 0) {
    const int xcd = t % 8, k = t / 8;
    g = xcd % groups;
    rb = xcd / groups + (8 / groups) * k;
  } else {
    g = t / rbs;
    rb = t % rbs;
  }
}

// Block-uniform result of a wait run by wave 0.
__device__ __forceinline__ bool block_wait(bool wave0_ok, int* s_flag) {
  if (threadIdx.x == 0) *s_flag = wave0_ok ? 1 : 0;
  __syncthreads();
  const bool ok = *s_flag != 0;
  __syncthreads();
  return ok;
}

// This block's results are stored (coherently): wait for them, then count
// the block in at `counter`; returns the counter's previous value (thread 0).
__device__ __forceinline__ uint32_t publish(uint32_t* counter) {
  lemoq_sync::wait_own_stores();
  __syncthreads();
  uint32_t prev = 0;
  if (threadIdx.x == 0)
    prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return prev;
}

template <int NSMAX, int KCH, int NP>
__global__ __launch_bounds__(256) void attn_layer_kernel(const LayerArgs a) {
  __shared__ lemoq_attn_fused::AttnFusedSmem<128, 4> sm;
  __shared__ __align__(16) uint16_t xs[KCH * 1024 > MO_COLS ? KCH * 1024 : MO_COLS];
  __shared__ float red[4];
  __shared__ int s_flag;
  const int G = gridDim.x, b = blockIdx.x;
  const int heads = a.at.heads, ns = a.at.ns;
  const int groups = heads / MO_HEADS;
  uint32_t* status = a.sync;

  // Loads that depend on nothing this launch computes go first: the first
  // o_proj tile's weight slices and, for a router block, its router rows, h
  // and the norm weight.
  OprojTile tile;
  int g0 = 0, rb0 = 0;
  if (b < a.n_tiles) {
    tile_coords(b, groups, a.row_blocks, a.n_tiles, g0, rb0);
    oproj_issue(a.mo, g0, rb0, tile);
  }
  RouterPre<KCH> pre;
  if (b < a.n_router) router_issue<KCH>(a.rr, b, pre);

  // A: split block (sp, h).
  const int h = b / ns, sp = b % ns;
  lemoq_attn_fused::attn_split_fused_block<128, 4, 3, true>(a.at, sp, h, sm);
  publish(line(a, 1 + h));

  // B: o_proj tiles b, b + G, ...
  for (int t = b; t < a.n_tiles; t += G) {
    int g = g0, rb = rb0;
    if (t != b) {
      tile_coords(t, groups, a.row_blocks, a.n_tiles, g, rb);
      oproj_issue(a.mo, g, rb, tile);
    }
    bool ok = true;
    if (threadIdx.x < 64)
      ok = lemoq_sync::wait_counts(line(a, 1 + g * MO_HEADS), MO_HEADS, (uint32_t)ns, status, a.limit_ticks);
    if (!block_wait(ok, &s_flag)) return;
    oproj_finish<NSMAX, true>(a.mo, tile, xs);
    publish(line(a, 1 + heads + t % kTileLines));
  }

  // C: router block b.
  if (b < a.n_router) {
    bool ok = true;
    if (threadIdx.x < 64) {
      const int k = threadIdx.x;  // lane k polls counter k: tiles t < n_tiles with t % 16 == k
      const uint32_t want = k < kTileLines ? (uint32_t)((a.n_tiles - k + kTileLines - 1) / kTileLines) : 0u;
      ok = lemoq_sync::wait_counts(line(a, 1 + heads), kTileLines, want, status, a.limit_ticks);
    }
    if (!block_wait(ok, &s_flag)) return;
    router_finish<KCH, NP, true>(a.rr, b, pre, xs, red);
    const uint32_t prev = publish(line(a, 1 + heads + kTileLines));
    if (threadIdx.x == 0 && prev == (uint32_t)(a.n_router - 1)) {
      // Every router block has passed its wait, so every tile passed its own:
      // no workgroup reads a counter any more.
      for (int i = 1; i <= heads + kTileLines + 1; ++i) lemoq_sync::st_u32(line(a, i), 0u);
    }
  }
}

__global__ __launch_bounds__(256) void sync_zero_kernel(uint32_t* w, int64_t n) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) w[i] = 0u;
}

bool overlaps(const void* x, int64_t nx, const void* y, int64_t ny) {
  const char* p = static_cast<const char*>(x);
  const char* q = static_cast<const char*>(y);
  return p < q + ny && q < p + nx;
}

template <int NSMAX, int KCH, int NP>
int resident_blocks(int device) {
  // Workgroups of this instance that can be resident at once on `device`
  // (cached per device; 0 when the query fails).
  static int cache[64];
  static bool known[64];
  if (device < 0 || device >= 64) return 0;
  if (!known[device]) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_layer_kernel<NSMAX, KCH, NP>, 256, 0) !=
            hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return 0;
    cache[device] = per_cu * cus;
    known[device] = true;
  }
  return cache[device];
}

template <int NSMAX, int KCH, int NP>
int launch_layer(const LayerArgs& a, int G, hipStream_t st) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return LEMOQ_ERR_UNSUPPORTED;
  if (resident_blocks<NSMAX, KCH, NP>(device) < G) return LEMOQ_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((attn_layer_kernel<NSMAX, KCH, NP>), dim3((unsigned)G), dim3(256), 0, st, a);
  LEMOQ_CHECK_LAUNCH();
}

template <int NSMAX, int KCH>
int dispatch_np(const LayerArgs& a, int np, int G, hipStream_t st) {
  switch (np) {
    case 1: return launch_layer<NSMAX, KCH, 1>(a, G, st);
    case 2: return launch_layer<NSMAX, KCH, 2>(a, G, st);
    case 4: return launch_layer<NSMAX, KCH, 4>(a, G, st);
    default: return launch_layer<NSMAX, KCH, 8>(a, G, st);
  }
}

}  // namespace

extern "C" int lemoq_attn_layer_check(int64_t heads, int64_t head_dim, int64_t num_splits, int64_t hidden,
                                      int64_t group, int64_t num_experts) {
  if (head_dim != MO_D || heads <= 0 || heads % MO_HEADS != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (hidden != 2048 && hidden != 4096) return LEMOQ_ERR_UNSUPPORTED;
  const int64_t HD = heads * head_dim, np = HD / MO_COLS;
  if (np != 1 && np != 2 && np != 4 && np != 8) return LEMOQ_ERR_UNSUPPORTED;
  if (num_splits <= 0 || num_splits > 64 || group <= 0 || group % 16 != 0 || HD % group != 0)
    return LEMOQ_ERR_SHAPE;
  const int64_t G = heads * num_splits;
  if (num_experts <= 0 || (num_experts + 3) / 4 > G) return LEMOQ_ERR_SHAPE;
  // lines 1 .. heads + 17; lemoq_moe_layer_w8 uses lines 64 and up
  if (1 + heads + kTileLines + 1 > 64) return LEMOQ_ERR_SHAPE;
  // every workgroup resident at once
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return LEMOQ_ERR_UNSUPPORTED;
  int cap = 0;
  const int kch = (int)(hidden / 1024);
  const bool small = num_splits <= 16;
#define LEMOQ_RES(NSM, KC, NPP) cap = resident_blocks<NSM, KC, NPP>(device)
  if (kch == 2) {
    if (small) { switch (np) { case 1: LEMOQ_RES(16, 2, 1); break; case 2: LEMOQ_RES(16, 2, 2); break; case 4: LEMOQ_RES(16, 2, 4); break; default: LEMOQ_RES(16, 2, 8); } }
    else { switch (np) { case 1: LEMOQ_RES(64, 2, 1); break; case 2: LEMOQ_RES(64, 2, 2); break; case 4: LEMOQ_RES(64, 2, 4); break; default: LEMOQ_RES(64, 2, 8); } }
  } else {
    if (small) { switch (np) { case 1: LEMOQ_RES(16, 4, 1); break; case 2: LEMOQ_RES(16, 4, 2); break; case 4: LEMOQ_RES(16, 4, 4); break; default: LEMOQ_RES(16, 4, 8); } }
    else { switch (np) { case 1: LEMOQ_RES(64, 4, 1); break; case 2: LEMOQ_RES(64, 4, 2); break; case 4: LEMOQ_RES(64, 4, 4); break; default: LEMOQ_RES(64, 4, 8); } }
  }
#undef LEMOQ_RES
  return cap >= G ? LEMOQ_OK : LEMOQ_ERR_UNSUPPORTED;
}

extern "C" int lemoq_attn_layer_i8(const uint16_t* qkv, int64_t heads, int64_t head_dim,
                                   const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                                   const uint16_t* cos_tab, const uint16_t* sin_tab, const int64_t* pos,
                                   int8_t* kc, uint16_t* ks, int8_t* vc, uint16_t* vs,
                                   int64_t code_head_stride, int64_t s_len, int64_t num_splits,
                                   float qk_scale, float* m, float* l, float* acc,
                                   const int8_t* o_codes, const uint16_t* o_scale, int64_t hidden,
                                   int64_t group, float* o_part, const uint16_t* h,
                                   const uint16_t* post_norm_w, const uint16_t* router_w,
                                   int64_t num_experts, uint16_t* h_out, uint16_t* xn_out,
                                   uint16_t* logits, uint32_t* sync, int64_t timeout_us, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !pos || !kc || !ks || !vc || !vs || !m ||
      !l || !acc || !o_codes || !o_scale || !o_part || !h || !post_norm_w || !router_w || !h_out ||
      !logits || !sync)
    return LEMOQ_ERR_NULL;
  if (timeout_us < 0) return LEMOQ_ERR_SHAPE;
  if (s_len <= 0 || s_len >= (int64_t(1) << 31) || code_head_stride < s_len * head_dim)
    return LEMOQ_ERR_SHAPE;
  const int rc = lemoq_attn_layer_check(heads, head_dim, num_splits, hidden, group, num_experts);
  if (rc) return rc;
  const int64_t HD = heads * head_dim;
  if (!lemoq_aligned16(qkv) || !lemoq_aligned16(kc) || !lemoq_aligned16(vc) || code_head_stride % 16 != 0 ||
      !lemoq_aligned16(o_codes) || !lemoq_aligned16(o_part) || !lemoq_aligned16(h) ||
      !lemoq_aligned16(post_norm_w) || !lemoq_aligned16(router_w) || !lemoq_aligned16(h_out) ||
      (xn_out && !lemoq_aligned16(xn_out)) || (reinterpret_cast<uintptr_t>(sync) & 255u) != 0)
    return LEMOQ_ERR_ALIGN;
  // Router blocks read h while router block 0 writes h_out.
  if (overlaps(h_out, hidden * 2, h, hidden * 2) || overlaps(h_out, hidden * 2, o_part, (HD / MO_COLS) * hidden * 4))
    return LEMOQ_ERR_SHAPE;
  LayerArgs a;
  a.at.qkv = qkv;
  a.at.qn_w = q_norm_w;
  a.at.kn_w = k_norm_w;
  a.at.eps = eps;
  a.at.cos_tab = cos_tab;
  a.at.sin_tab = sin_tab;
  a.at.pos = pos;
  a.at.kc = kc;
  a.at.ks = ks;
  a.at.vc = vc;
  a.at.vs = vs;
  a.at.code_head_stride = code_head_stride;
  a.at.s_len = s_len;
  a.at.heads = (int)heads;
  a.at.ns = (int)num_splits;
  a.at.qk_scale = qk_scale;
  a.at.m_out = m;
  a.at.l_out = l;
  a.at.acc_out = acc;
  a.mo.m = m;
  a.mo.l = l;
  a.mo.acc = acc;
  a.mo.NS = (int)num_splits;
  a.mo.codes = o_codes;
  a.mo.scale = o_scale;
  a.mo.N = hidden;
  a.mo.HD = (int)HD;
  a.mo.group = (int)group;
  a.mo.part = o_part;
  a.rr.part = o_part;
  a.rr.h = h;
  a.rr.norm_w = post_norm_w;
  a.rr.eps = eps;
  a.rr.H = (int)hidden;
  a.rr.rw = router_w;
  a.rr.E = (int)num_experts;
  a.rr.h_out = h_out;
  a.rr.xn_out = xn_out;
  a.rr.logits = logits;
  a.sync = sync;
  a.limit_ticks = (uint64_t)timeout_us * 100u;  // s_memrealtime runs at 100 MHz
  a.row_blocks = (int)(hidden / MO_ROWS);
  a.n_tiles = a.row_blocks * (int)(heads / MO_HEADS);
  a.n_router = (int)((num_experts + 3) / 4);
  const int G = (int)(heads * num_splits);
  const int np = (int)(HD / MO_COLS);
  hipStream_t st = lemoq_stream(stream);
  if (hidden == 2048)
    return num_splits <= 16 ? dispatch_np<16, 2>(a, np, G, st) : dispatch_np<64, 2>(a, np, G, st);
  return num_splits <= 16 ? dispatch_np<16, 4>(a, np, G, st) : dispatch_np<64, 4>(a, np, G, st);
}

extern "C" int lemoq_sync_reset(uint32_t* sync, void* stream) {
  if (!sync) return LEMOQ_ERR_NULL;
  hipLaunchKernelGGL(sync_zero_kernel, dim3(8), dim3(256), 0, lemoq_stream(stream), sync,
                     (int64_t)LEMOQ_SYNC_WORDS);
  LEMOQ_CHECK_LAUNCH();
}
