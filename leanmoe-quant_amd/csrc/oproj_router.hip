// The attention-output half of an OLMoE decoder layer at batch 1 in two
// launches instead of three (merge, o_proj, router); the device parts are in
// oproj_router.h.
#include "oproj_router.h"

namespace {

using namespace lemoq_oproj;

template <int NSMAX>
__global__ __launch_bounds__(256) void merge_oproj_kernel(const MergeOprojArgs a) {
  __shared__ __align__(16) uint16_t xs[MO_COLS];
  int g, rb;
  oproj_tile_of_block(g, rb);
  OprojTile t;
  oproj_issue(a, g, rb, t);
  LEMOQ_LOADS_ISSUED();  // the weight stream first, then the merge inputs
  oproj_finish<NSMAX>(a, t, xs);
}

template <int NSMAX>
__global__ __launch_bounds__(256) void merge_oproj_q4_kernel(const MergeOprojArgs a) {
  __shared__ __align__(16) uint16_t xs[MO_COLS];
  int g, rb;
  oproj_tile_of_block(g, rb);
  OprojTileQ4 t;
  oproj_issue_q4(a, g, rb, t);
  LEMOQ_LOADS_ISSUED();  // the weight stream first, then the merge inputs
  oproj_finish_q4<NSMAX>(a, t, xs);
}

template <int KCH, int NP>
__global__ __launch_bounds__(256) void router_resid_kernel(const RouterResidArgs a) {
  __shared__ __align__(16) uint16_t xs[KCH * 1024];
  __shared__ float red[4];
  RouterPre<KCH> p;
  router_issue<KCH>(a, blockIdx.x, p);
  router_finish<KCH, NP>(a, blockIdx.x, p, xs, red);
}

bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
  const char* x = static_cast<const char*>(a);
  const char* y = static_cast<const char*>(b);
  return x < y + nb && y < x + na;
}

}  // namespace

namespace {

int merge_oproj(const float* m, const float* l, const float* acc, int64_t heads, int64_t num_splits,
                int64_t head_dim, const int8_t* codes, const uint16_t* scale, int64_t N, int64_t group, float* part,
                void* stream, int bits) {
  if (!m || !l || !acc || !codes || !scale || !part) return LEMOQ_ERR_NULL;
  if (heads <= 0 || num_splits <= 0 || N <= 0 || group <= 0) return LEMOQ_ERR_SHAPE;
  if (head_dim != MO_D || heads % MO_HEADS != 0) return LEMOQ_ERR_UNSUPPORTED;
  if (num_splits > 64 || N % MO_ROWS != 0 || N / MO_ROWS > 0x7fffffff || heads / MO_HEADS > 65535)
    return LEMOQ_ERR_SHAPE;
  const int64_t HD = heads * head_dim;
  // a lane's slice (16 codes at 8 bits, 32 at 4) lies inside one scale group
  if (group % (bits == 4 ? 32 : 16) != 0 || HD % group != 0 || HD > 0x7fffffff) return LEMOQ_ERR_SHAPE;
  if (!lemoq_aligned16(codes)) return LEMOQ_ERR_ALIGN;
  MergeOprojArgs a;
  a.m = m;
  a.l = l;
  a.acc = acc;
  a.NS = (int)num_splits;
  a.codes = codes;
  a.scale = scale;
  a.N = N;
  a.HD = (int)HD;
  a.group = (int)group;
  a.part = part;
  const dim3 grid((unsigned)(N / MO_ROWS), (unsigned)(heads / MO_HEADS));
  hipStream_t st = lemoq_stream(stream);
  if (bits == 4) {
    if (num_splits <= 16)
      hipLaunchKernelGGL((merge_oproj_q4_kernel<16>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((merge_oproj_q4_kernel<64>), grid, dim3(256), 0, st, a);
  } else {
    if (num_splits <= 16)
      hipLaunchKernelGGL((merge_oproj_kernel<16>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((merge_oproj_kernel<64>), grid, dim3(256), 0, st, a);
  }
  LEMOQ_CHECK_LAUNCH();
}

}  // namespace

extern "C" int lemoq_attn_merge_o_proj_w8(const float* m, const float* l, const float* acc,
                                          int64_t heads, int64_t num_splits, int64_t head_dim,
                                          const int8_t* codes, const uint16_t* scale, int64_t N,
                                          int64_t group, float* part, void* stream) {
  return merge_oproj(m, l, acc, heads, num_splits, head_dim, codes, scale, N, group, part, stream, 8);
}

extern "C" int lemoq_attn_merge_o_proj_w4(const float* m, const float* l, const float* acc,
                                          int64_t heads, int64_t num_splits, int64_t head_dim,
                                          const uint8_t* codes, const uint16_t* scale, int64_t N,
                                          int64_t group, float* part, void* stream) {
  return merge_oproj(m, l, acc, heads, num_splits, head_dim, reinterpret_cast<const int8_t*>(codes), scale, N,
                     group, part, stream, 4);
}

extern "C" int lemoq_router_logits_resid(const float* part, int64_t n_part, const uint16_t* h,
                                         const uint16_t* norm_w, float eps, int64_t hidden,
                                         const uint16_t* router_w, int64_t E, uint16_t* h_out,
                                         uint16_t* xn_out, uint16_t* logits, void* stream) {
  if (!part || !h || !norm_w || !router_w || !h_out || !logits) return LEMOQ_ERR_NULL;
  if (E <= 0 || E > 4 * 65535 || n_part <= 0) return LEMOQ_ERR_SHAPE;
  if (hidden != 2048 && hidden != 4096) return LEMOQ_ERR_UNSUPPORTED;
  if (n_part != 1 && n_part != 2 && n_part != 4 && n_part != 8) return LEMOQ_ERR_UNSUPPORTED;
  if (!lemoq_aligned16(part) || !lemoq_aligned16(h) || !lemoq_aligned16(norm_w) ||
      !lemoq_aligned16(router_w) || !lemoq_aligned16(h_out) || (xn_out && !lemoq_aligned16(xn_out)))
    return LEMOQ_ERR_ALIGN;
  // Every block reads h while block 0 writes h_out: they must not share memory.
  if (overlaps(h_out, hidden * 2, h, hidden * 2) || overlaps(h_out, hidden * 2, part, n_part * hidden * 4))
    return LEMOQ_ERR_SHAPE;
  RouterResidArgs a;
  a.part = part;
  a.h = h;
  a.norm_w = norm_w;
  a.eps = eps;
  a.H = (int)hidden;
  a.rw = router_w;
  a.E = (int)E;
  a.h_out = h_out;
  a.xn_out = xn_out;
  a.logits = logits;
  const dim3 grid((unsigned)((E + 3) / 4));
  hipStream_t st = lemoq_stream(stream);
#define LEMOQ_RR_CASE(KK, PP) \
  hipLaunchKernelGGL((router_resid_kernel<KK, PP>), grid, dim3(256), 0, st, a)
  if (hidden == 2048) {
    switch (n_part) {
      case 1: LEMOQ_RR_CASE(2, 1); break;
      case 2: LEMOQ_RR_CASE(2, 2); break;
      case 4: LEMOQ_RR_CASE(2, 4); break;
      default: LEMOQ_RR_CASE(2, 8); break;
    }
  } else {
    switch (n_part) {
      case 1: LEMOQ_RR_CASE(4, 1); break;
      case 2: LEMOQ_RR_CASE(4, 2); break;
      case 4: LEMOQ_RR_CASE(4, 4); break;
      default: LEMOQ_RR_CASE(4, 8); break;
    }
  }
#undef LEMOQ_RR_CASE
  LEMOQ_CHECK_LAUNCH();
}
