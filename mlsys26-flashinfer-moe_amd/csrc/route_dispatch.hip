// Routing and dispatch for the fused MoE layer (gfx950).
//
// The DeepSeek-V3 no-aux grouped routing (kernel.py:428-542) runs with branch-free DPP
// reductions: up to 256 tokens one token per wavefront (route_wide_kernel: 4 experts per lane,
// the shortest dependent chain per token), above that sixteen lanes per token and four
// tokens per wavefront (route_kernel, which also records per-work-group histograms and ranks
// for the multi-work-group dispatch). Dispatch then histograms the local assignments, scans
// them into CSR offsets, builds the GEMM work list and places every assignment in its bucket:
//   T <= 256 (or given top-k lists): route_wide_kernel -> dispatch_small_kernel, which does the
//             whole dispatch in one work-group, in LDS (up to 64 tokens moe_fp8_run rebuilds the
//             dispatch inside GEMM1 instead);
//   larger T: route_kernel (also per work-group histograms and ranks) -> place_kernel (above
//             16384 tokens with block_scan_kernel between them, which keeps the cost linear in T)
//             (each work-group reduces the histograms it needs). No kernel synchronises
//             across work-groups.
//
// The order inside an expert's bucket is ascending token (then slot), i.e. a stable sort
// by expert of the flat top-k list; the reference's atomic scatter (kernel.py:288-324)
// produces the same buckets in a run-dependent order.
#include "moe_internal.h"
#include "moe_device.h"

namespace moe {

namespace {

__device__ __forceinline__ float load_bias(const void* bias, int dtype, int i) {
  if (dtype == MOE_FP8_BIAS_F32) return reinterpret_cast<const float*>(bias)[i];
  const uint16_t h = reinterpret_cast<const uint16_t*>(bias)[i];
  if (dtype == MOE_FP8_BIAS_BF16) return __uint_as_float((uint32_t)h << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

// Multiset top-2 merge: (a1 >= a2) and (b1 >= b2) -> the two largest of the four.
__device__ __forceinline__ void top2_merge(float& m1, float& m2, float o1, float o2) {
  const float n1 = fmaxf(m1, o1);
  const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
  m1 = n1;
  m2 = n2;
}

// DPP lane permutations (within rows of 16 lanes).
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15-i within 16

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}

// Argmax keys of the routing: a larger fp32 value wins, then the lower expert index (the
// "lowest index on ties" rule of kernel.py:499 and :525): key = ordered(v) << 32 | 0xFFFF - e.
__device__ __forceinline__ int key_index(uint64_t key) { return 0xFFFF - (int)(key & 0xFFFFu); }

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Order-preserving map of a float to an unsigned key (after -0 -> +0, so equal values tie):
// a > b as floats <=> ordered(a) > ordered(b).
__device__ __forceinline__ uint32_t ordered(float v) {
  const uint32_t u = __float_as_uint(v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
constexpr uint32_t kOrderedNegInf = 0x007FFFFFu;   // ordered(-inf)

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// 1 if group pg with score pv ranks before group g with score gs in the group selection
// (larger score first, lower index on ties); pv, pg come from the lane ROT lanes away
// within the 16-lane row.
template <int ROT>
__device__ __forceinline__ int group_beats(float gs, int g) {
  constexpr int kCtrl = 0x120 + ROT;   // DPP row_ror:ROT
  const float pv = __int_as_float(dpp_i32<kCtrl>(__float_as_int(gs)));
  const int pg = dpp_i32<kCtrl>(g);
  return (pv > gs || (pv == gs && pg < g)) ? 1 : 0;
}

// Token routed by this lane's 16-lane row when the wavefront routes tokens t0 .. t0+3.
__device__ __forceinline__ int route_row(int t0, int T) {
  return min(t0 + (lane_id() >> 4), T - 1);   // rows past the end recompute the last token
}
__device__ __forceinline__ void load_logits(const RouteParams& p, int t0, float4 (&lg)[4]) {
  const float4* lp = reinterpret_cast<const float4*>(p.logits + (size_t)route_row(t0, p.T) * kExpertsGlobal +
                                                     16 * (lane_id() & 15));
#pragma unroll
  for (int i = 0; i < 4; ++i) lg[i] = lp[i];
}
// Routing of 4 tokens by one wavefront (kernel.py:428-542). Token q = lane/16 of the
// wavefront is t0 + q; lane r = lane%16 of its row holds experts 16r..16r+15, so group g
// (32 experts) is lanes 2g, 2g+1. The lane's 16 logits come in `lg` (loaded by the caller
// before the bias staging barrier, so that the two loads overlap). Returns in lanes r < 8
// the expert of top-k slot r (in selection order) and its weight; other lanes return -1.
__device__ __forceinline__ int route_wave(const RouteParams& p, const float* s_bias, int t0, const float4 (&lg)[4],
                                          float& w_out) {
  const int lane = lane_id();
  const int r = lane & 15;
  const int t = route_row(t0, p.T);
  const float4* bp = reinterpret_cast<const float4*>(s_bias + 16 * r);
  float s[16], b[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 x = lg[i], c = bp[i];
    const float xs[4] = {x.x, x.y, x.z, x.w}, cs[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s[4 * i + j] = sigmoid_f32(xs[j]);        // kernel.py:466
      b[4 * i + j] = s[4 * i + j] + cs[j];      // kernel.py:467
    }
  }
  // Group score = sum of the two largest biased scores of the group (kernel.py:479-488):
  // top-2 of the lane's 16 (median-of-three keeps the runner-up), then of the lane pair.
  float m1 = fmaxf(b[0], b[1]), m2 = fminf(b[0], b[1]);
#pragma unroll
  for (int i = 2; i < 16; ++i) {
    const float n2 = __builtin_amdgcn_fmed3f(m1, m2, b[i]);
    m1 = fmaxf(m1, b[i]);
    m2 = n2;
  }
  top2_merge(m1, m2, dpp_f32<kDppXor1>(m1), dpp_f32<kDppXor1>(m2));
  const float gs = m1 + m2;
  // Keep the 4 best groups (kernel.py:495-501): a group is kept iff fewer than 4 groups
  // rank before it. The seven other groups of the row are 2, 4, ..., 14 lanes away.
  const int g = r >> 1;
  const int rank = group_beats<2>(gs, g) + group_beats<4>(gs, g) + group_beats<6>(gs, g) +
                   group_beats<8>(gs, g) + group_beats<10>(gs, g) + group_beats<12>(gs, g) +
                   group_beats<14>(gs, g);
  const bool kept = rank < kTopKGroup;

  // Top-8 experts of the kept groups by biased score, lowest index on ties (kernel.py:515-534):
  // 8 rounds of (argmax inside the lane, argmax across the row on 64-bit keys
  // (score key << 32 | 0xFFFF - expert), removal of the winner from its lane).
  uint32_t c[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) c[i] = kept ? ordered(b[i]) : kOrderedNegInf;
  const uint32_t lo_base = 0xFFFFu - 16u * (uint32_t)r;
  int my_id = -1;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    uint32_t v8[8], i8[8], v4[4], i4[4], v2[2], i2[2];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool hi = c[2 * j + 1] > c[2 * j];
      v8[j] = hi ? c[2 * j + 1] : c[2 * j];
      i8[j] = hi ? 2 * j + 1 : 2 * j;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool hi = v8[2 * j + 1] > v8[2 * j];
      v4[j] = hi ? v8[2 * j + 1] : v8[2 * j];
      i4[j] = hi ? i8[2 * j + 1] : i8[2 * j];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bool hi = v4[2 * j + 1] > v4[2 * j];
      v2[j] = hi ? v4[2 * j + 1] : v4[2 * j];
      i2[j] = hi ? i4[2 * j + 1] : i4[2 * j];
    }
    const bool hi = v2[1] > v2[0];
    const uint32_t bv = hi ? v2[1] : v2[0];
    const uint32_t bi = hi ? i2[1] : i2[0];
    uint64_t key = ((uint64_t)bv << 32) | (lo_base - bi);
    key = max_u64(key, dpp_u64<kDppXor1>(key));
    key = max_u64(key, dpp_u64<kDppXor2>(key));
    key = max_u64(key, dpp_u64<kDppHalfMirror>(key));
    key = max_u64(key, dpp_u64<kDppMirror>(key));
    const int e = key_index(key);
    my_id = (r == k) ? e : my_id;
    // the winner's score becomes -inf (kernel.py:534), not less: once fewer than 8 finite
    // scores remain, every -inf entry ties, the chosen ones included, and the lowest index
    // wins again (a token can then name one expert several times, as the reference does)
    const uint32_t drop = ((e >> 4) == r) ? (uint32_t)(e & 15) : 16u;
#pragma unroll
    for (int i = 0; i < 16; ++i) c[i] = (drop == (uint32_t)i) ? kOrderedNegInf : c[i];
  }
  // Weights from the unbiased scores, renormalised in selection order and scaled
  // (kernel.py:537-538): w = s / (s_0 + ... + s_7 + 1e-20) * rsf. Lane r < 8 recomputes
  // the score of its expert; every lane then sums the row's eight in order.
  const float sv = (r < kTopK) ? sigmoid_f32(p.logits[(size_t)t * kExpertsGlobal + my_id]) : 0.0f;
  const int row0 = lane & 48;
  float sum = __shfl(sv, row0);
#pragma unroll
  for (int k = 1; k < kTopK; ++k) sum = sum + __shfl(sv, row0 | k);
  sum = sum + 1e-20f;
  w_out = __fdiv_rn(sv, sum) * p.rsf;
  return r < kTopK ? my_id : -1;
}

// DPP row broadcasts across the 16-lane rows of a wavefront (GFX9): lane 15 of each row to
// the next row (rows 1 and 3 take it), lane 31 to rows 2 and 3.
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_u64_rows(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROW_MASK, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROW_MASK, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}

// Routing of token t by one wavefront (kernel.py:428-542), for small batches: lane l holds
// experts 4l..4l+3, so group g (32 experts) is lanes 8g..8g+7, and every lane does a quarter
// of route_wave's per-token work. The selections are route_wave's: the same argmax keys, the
// group score as the sum of the group's two largest biased scores, the kept groups by (score,
// lower index), the weights summed in selection order with the same fp32 operations, so
// the top-k lists are bit-identical. `lg` holds the lane's four logits. Returns in lanes
// k < 8 the expert of top-k slot k and its weight; other lanes return -1.
__device__ __forceinline__ int route_wide(const RouteParams& p, const float* s_bias, int t, const float4 lg,
                                          float& w_out) {
  const int lane = lane_id();
  const float4 cb = reinterpret_cast<const float4*>(s_bias)[lane];
  const float xs[4] = {lg.x, lg.y, lg.z, lg.w}, cs[4] = {cb.x, cb.y, cb.z, cb.w};
  float b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) b[j] = sigmoid_f32(xs[j]) + cs[j];   // kernel.py:466-467
  // group score (kernel.py:479-488): top-2 of the lane's four, then of the group's 8 lanes
  float m1 = fmaxf(b[0], b[1]), m2 = fminf(b[0], b[1]);
#pragma unroll
  for (int i = 2; i < 4; ++i) {
    const float n2 = __builtin_amdgcn_fmed3f(m1, m2, b[i]);
    m1 = fmaxf(m1, b[i]);
    m2 = n2;
  }
  top2_merge(m1, m2, dpp_f32<kDppXor1>(m1), dpp_f32<kDppXor1>(m2));
  top2_merge(m1, m2, dpp_f32<kDppXor2>(m1), dpp_f32<kDppXor2>(m2));
  top2_merge(m1, m2, dpp_f32<kDppHalfMirror>(m1), dpp_f32<kDppHalfMirror>(m2));
  const float gs = m1 + m2;
  // the 4 best groups (kernel.py:495-501): the eight scores are wave-uniform (lane 8h holds
  // group h's), and a group is kept iff fewer than 4 groups rank before it
  const int g = lane >> 3;
  int rank = 0;
#pragma unroll
  for (int h = 0; h < kNGroup; ++h) {
    const float hs = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gs), 8 * h));
    rank += (hs > gs || (hs == gs && h < g)) ? 1 : 0;
  }
  const bool kept = rank < kTopKGroup;
  // top-8 experts of the kept groups (kernel.py:515-534): 8 rounds of (argmax inside the
  // lane, argmax of the 64-bit keys across the wavefront, removal of the winner)
  uint32_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = kept ? ordered(b[i]) : kOrderedNegInf;
  const uint32_t lo_base = 0xFFFFu - 4u * (uint32_t)lane;
  int my_id = -1;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    const bool h01 = c[1] > c[0], h23 = c[3] > c[2];
    const uint32_t v01 = h01 ? c[1] : c[0], v23 = h23 ? c[3] : c[2];
    const uint32_t i01 = h01 ? 1u : 0u, i23 = h23 ? 3u : 2u;
    const bool hi = v23 > v01;
    uint64_t key = ((uint64_t)(hi ? v23 : v01) << 32) | (lo_base - (hi ? i23 : i01));
    key = max_u64(key, dpp_u64<kDppXor1>(key));
    key = max_u64(key, dpp_u64<kDppXor2>(key));
    key = max_u64(key, dpp_u64<kDppHalfMirror>(key));
    key = max_u64(key, dpp_u64<kDppMirror>(key));
    key = max_u64(key, dpp_u64_rows<kDppRowBcast15, 0xA>(key));
    key = max_u64(key, dpp_u64_rows<kDppRowBcast31, 0xC>(key));
    // lane 63 holds the wavefront's largest key
    const uint32_t klo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, 63);
    const int e = key_index((uint64_t)klo);
    my_id = (lane == k) ? e : my_id;
    // the winner drops to -inf, where it ties with the other -inf entries (kernel.py:534)
    const uint32_t drop = ((e >> 2) == lane) ? (uint32_t)(e & 3) : 4u;
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = (drop == (uint32_t)i) ? kOrderedNegInf : c[i];
  }
  // weights (kernel.py:537-538), as route_wave: w = s / (s_0 + ... + s_7 + 1e-20) * rsf
  const float sv = (lane < kTopK) ? sigmoid_f32(p.logits[(size_t)t * kExpertsGlobal + my_id]) : 0.0f;
  float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv), 0));
#pragma unroll
  for (int k = 1; k < kTopK; ++k) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv), k));
  sum = sum + 1e-20f;
  w_out = __fdiv_rn(sv, sum) * p.rsf;
  return lane < kTopK ? my_id : -1;
}

__device__ __forceinline__ int local_of(int id, int offset) {
  const int le = id - offset;
  return (le >= 0 && le < kExpertsLocal) ? le : -1;
}

// Router bias (fp32, bf16 or fp16) -> fp32 in LDS; the whole work-group calls this.
__device__ __forceinline__ void stage_bias(const RouteParams& p, float* s_bias) {
  if (!p.skip_routing && threadIdx.x < kExpertsGlobal) s_bias[threadIdx.x] = load_bias(p.bias, p.bias_dtype, threadIdx.x);
  __syncthreads();
}

// Stable rank of each thread's slot among the work-group's slots with the same local expert
// (lower thread index first), plus per-expert counts. Up to 16 wavefronts, one slot per
// thread (le < 0: not local). s_wcnt is [16][32] scratch; s_cnt receives the counts.
__device__ __forceinline__ int block_rank(int le, int nwaves, int (*s_wcnt)[kExpertsLocal], int* s_cnt) {
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const uint64_t lt = lanemask_lt();
  int rank = 0, cnt = 0;
#pragma unroll 4
  for (int e = 0; e < kExpertsLocal; ++e) {
    const uint64_t m = __ballot(le == e);
    if (le == e) rank = __popcll(m & lt);
    if (lane == e) cnt = __popcll(m);
  }
  if (lane < kExpertsLocal) s_wcnt[wave][lane] = cnt;
  __syncthreads();
  if (threadIdx.x < kExpertsLocal) {
    int run = 0;
    for (int w = 0; w < nwaves; ++w) {
      const int v = s_wcnt[w][threadIdx.x];
      s_wcnt[w][threadIdx.x] = run;
      run += v;
    }
    s_cnt[threadIdx.x] = run;
  }
  __syncthreads();
  return le >= 0 ? rank + s_wcnt[wave][le] : 0;
}

// Lanes 0..31 of one wavefront, lane e holding expert e's total: CSR offsets, counters and
// the GEMM work list (kernel.py:357-360 and :384-407 build the equivalents). Each expert's
// rows are cut into runs of at most rows_per_item rows; above 32 rows the runs are balanced
// (equal sizes rounded up to 16). Item = (expert, first row, rows,
// first item of the expert | items of the expert << 16).
__device__ __forceinline__ void finish_counts(const RouteParams& p, int e, int run, int* s_start) {
  int incl = run;
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) {
    const int o = __shfl_up(incl, off, 32);
    if (e >= off) incl += o;
  }
  p.expert_count[e] = run;
  p.expert_start[e + 1] = incl;
  s_start[e + 1] = incl;
  if (e == 0) { p.expert_start[0] = 0; s_start[0] = 0; }
  if (e == kExpertsLocal - 1) p.counters[kCtrAssign] = incl;
  const int bm = p.rows_per_item;
  int chunk = bm;
  if (bm > 32 && run > 0) {
    const int nmax = (run + bm - 1) / bm;
    chunk = min(bm, (((run + nmax - 1) / nmax) + 15) & ~15);
  }
  const int nch = (run + chunk - 1) / chunk;
  int ich = nch;
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) {
    const int o = __shfl_up(ich, off, 32);
    if (e >= off) ich += o;
  }
  const int first = ich - nch;
  const int start = incl - run;
  for (int c = 0; c < nch; ++c) {
    int4 it;
    it.x = e;
    it.y = start + c * chunk;
    it.z = min(chunk, run - c * chunk);
    it.w = first | (nch << 16);
    reinterpret_cast<int4*>(p.work_items)[first + c] = it;
  }
  if (e == kExpertsLocal - 1) p.counters[kCtrItems] = ich;
  // The order in which the tile kernels' per-XCD lists visit the experts: by descending item
  // rows (ties by expert index), experts without rows last. Their claim counters restart.
  const int key = nch > 0 ? min(chunk, run) : 0;
  int rank = 0;
  for (int o = 0; o < kExpertsLocal; ++o) {
    const int ko = __shfl(key, o, 32);
    rank += (ko > key || (ko == key && o < e)) ? 1 : 0;
  }
  p.counters[kCtrOrder + rank] = first | (nch << 16);
  p.counters[kCtrClaim + e] = 0;
  if (e < 2) p.counters[kCtrLeft + e] = 0;
}

}  // namespace

// Routing (or, on given top-k lists, loading) of 16 tokens per work-group of 4 wavefronts for
// the dispatch of large batches: the work-group also records every token's local count, the
// stable rank of each local slot among its 128 slots and its expert histogram.
constexpr int kRouteWaves = kRouteTokensPerBlock / 4;

__global__ __launch_bounds__(kRouteWaves * 64) void route_kernel(RouteParams p) {
  __shared__ __attribute__((aligned(16))) float s_bias[kExpertsGlobal];
  __shared__ int s_le[kRouteTokensPerBlock * kTopK];
  __shared__ int s_wcnt[16][kExpertsLocal];
  __shared__ int s_cnt[kExpertsLocal];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int r = lane & 15;
  const int tw = blockIdx.x * kRouteTokensPerBlock + wave * 4;   // first token of the wavefront
  const int t = tw + (lane >> 4);                                 // token of this lane's row
  const bool slot_lane = t < p.T && r < kTopK;                    // lane holds slot t*8 + r
  float4 lg[4];
  if (!p.skip_routing) load_logits(p, tw, lg);
  stage_bias(p, s_bias);
  int id = -1;
  float w = 0.f;
  if (!p.skip_routing) {
    id = route_wave(p, s_bias, tw, lg, w);
    if (slot_lane) {
      p.topk_ids[t * kTopK + r] = id;
      p.topk_w[t * kTopK + r] = w;
    }
  } else if (slot_lane) {
    id = p.topk_ids[t * kTopK + r];
  }
  {
    const int le = slot_lane ? local_of(id, p.offset) : -1;
    const uint64_t m = __ballot(le >= 0);
    if (r == 0 && t < p.T) p.token_nlocal[t] = __popcll((m >> (lane & 48)) & 0xFFull);
    if (r < kTopK) s_le[(wave * 4 + (lane >> 4)) * kTopK + r] = le;
    __syncthreads();
    // the 128 slots of the work-group are held by threads 0..127 (wavefronts 0 and 1)
    const int my_le = tid < kRouteTokensPerBlock * kTopK ? s_le[tid] : -1;
    const int rank = block_rank(my_le, kRouteWaves, s_wcnt, s_cnt);
    const int slot = blockIdx.x * kRouteTokensPerBlock * kTopK + tid;
    if (my_le >= 0) p.slot_rank[slot] = rank;
    if (tid < kExpertsLocal) p.block_count[blockIdx.x * kExpertsLocal + tid] = s_cnt[tid];
  }
}

// Dispatch of up to kRouteThreads slots held one per thread (slot tid = token tid/8, top-k
// position tid%8; le < 0: not a local expert): local counts, stable ranks, CSR offsets, the
// work list and the placement. The whole work-group calls this.
__device__ __forceinline__ void dispatch_slots(const RouteParams& p, int le, float w, int nslots,
                                               int (*s_wcnt)[kExpertsLocal], int* s_cnt, int* s_start) {
  const int tid = threadIdx.x;
  // the 8 slots of token tid/8 are 8 consecutive lanes, so one ballot gives every token's
  // local count
  const uint64_t m = __ballot(le >= 0);
  if ((tid & 7) == 0 && tid < nslots) p.token_nlocal[tid >> 3] = __popcll((m >> (lane_id() & 56)) & 0xFFull);
  const int r = block_rank(le, kRouteThreads / 64, s_wcnt, s_cnt);
  if (tid < kExpertsLocal) finish_counts(p, tid, s_cnt[tid], s_start);
  __syncthreads();
  if (le >= 0) {
    const int pos = s_start[le] + r;
    p.sorted_token[pos] = tid >> 3;
    p.sorted_weight[pos] = w;
    p.sorted_slot[pos] = tid;
  }
}

// Routing of up to kWideRouteTokens tokens, one token per wavefront and four per work-group
// (route_wide): top-k lists only, the dispatch follows in its own kernel or in GEMM1.
__global__ __launch_bounds__(256) void route_wide_kernel(RouteParams p) {
  __shared__ __attribute__((aligned(16))) float s_bias[kExpertsGlobal];
  const int lane = lane_id();
  const int tw = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int t = min(tw, p.T - 1);   // wavefronts past the end recompute the last token
  const float4 lg = reinterpret_cast<const float4*>(p.logits + (size_t)t * kExpertsGlobal)[lane];
  stage_bias(p, s_bias);
  float w = 0.f;
  const int id = route_wide(p, s_bias, t, lg, w);
  if (tw < p.T && lane < kTopK) {
    p.topk_ids[t * kTopK + lane] = id;
    p.topk_w[t * kTopK + lane] = w;
  }
}

// Dispatch of small batches (T <= kSinglePassTokens) in one work-group, from the top-k
// lists in the workspace: local counts, stable ranks (1024 slots at a time), CSR offsets,
// the work list and the placement, without leaving the work-group.
__global__ __launch_bounds__(kRouteThreads) void dispatch_small_kernel(RouteParams p) {
  __shared__ int s_le[kSinglePassTokens * kTopK];
  __shared__ int s_rank[kSinglePassTokens * kTopK];
  __shared__ float s_w[kSinglePassTokens * kTopK];
  __shared__ int s_wcnt[16][kExpertsLocal];
  __shared__ int s_cnt[kExpertsLocal];
  __shared__ int s_base[kExpertsLocal];
  __shared__ int s_start[kExpertsLocal + 1];

  const int tid = threadIdx.x;
  const int nslots = p.T * kTopK;
  if (nslots <= kRouteThreads) {
    // one slot per thread, kept in registers
    const int le = tid < nslots ? local_of(p.topk_ids[tid], p.offset) : -1;
    const float w = tid < nslots ? p.topk_w[tid] : 0.f;
    dispatch_slots(p, le, w, nslots, s_wcnt, s_cnt, s_start);
    return;
  }
  for (int slot = tid; slot < nslots; slot += kRouteThreads) {
    s_le[slot] = local_of(p.topk_ids[slot], p.offset);
    s_w[slot] = p.topk_w[slot];
  }
  if (tid < kExpertsLocal) s_base[tid] = 0;
  __syncthreads();
  for (int t = tid; t < p.T; t += kRouteThreads) {
    int n = 0;
#pragma unroll
    for (int k = 0; k < kTopK; ++k) n += s_le[t * kTopK + k] >= 0 ? 1 : 0;
    p.token_nlocal[t] = n;
  }
  for (int c0 = 0; c0 < nslots; c0 += kRouteThreads) {
    const int slot = c0 + tid;
    const int le = slot < nslots ? s_le[slot] : -1;
    const int r = block_rank(le, kRouteThreads / 64, s_wcnt, s_cnt);
    if (le >= 0) s_rank[slot] = s_base[le] + r;
    __syncthreads();
    if (tid < kExpertsLocal) s_base[tid] += s_cnt[tid];
    __syncthreads();
  }
  if (tid < kExpertsLocal) finish_counts(p, tid, s_base[tid], s_start);
  __syncthreads();
  for (int slot = tid; slot < nslots; slot += kRouteThreads) {
    const int le = s_le[slot];
    if (le < 0) continue;
    const int pos = s_start[le] + s_rank[slot];
    p.sorted_token[pos] = slot / kTopK;
    p.sorted_weight[pos] = s_w[slot];
    p.sorted_slot[pos] = slot;
  }
}

// Large batches, step 2: each local slot to its bucket position. Every work-group reduces the
// routing work-groups' histograms itself (no scan launch in between): thread (j, e) sums the
// counts of expert e over the blocks b = j mod kPlaceGroups, both over the blocks before its
// own (its exclusive prefix) and over all of them (the expert's total), kScanBatch loads in
// flight at a time; the partial sums meet in LDS. Work-group 0 also writes the CSR offsets,
// the counters and the work list (finish_counts); every work-group derives the same offsets.
constexpr int kScanBatch = 16;
constexpr int kPlaceThreads = 512;
constexpr int kPlaceGroups = kPlaceThreads / kExpertsLocal;   // 16
static_assert(kRouteTokensPerBlock * kTopK <= kPlaceThreads, "one slot per thread");

// SCANNED (batches of more than kPlaceDirectBlocks routing work-groups): block_scan_kernel has
// already turned block_count into per-work-group exclusive prefixes and written the CSR
// offsets, so that each work-group reads its 32 prefixes instead of reducing every
// histogram (which costs O(work-groups^2) in all).
template <bool SCANNED>
__global__ __launch_bounds__(kPlaceThreads) void place_kernel(RouteParams p) {
  __shared__ int s_pre[kPlaceGroups][kExpertsLocal];
  __shared__ int s_tot[kPlaceGroups][kExpertsLocal];
  __shared__ int s_prefix[kExpertsLocal];
  __shared__ int s_start[kExpertsLocal + 1];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int nb = p.nblocks;
  // this thread's slot, loaded before the reduction so that the loads overlap it
  const int s = b * kRouteTokensPerBlock * kTopK + tid;
  const bool has_slot = tid < kRouteTokensPerBlock * kTopK && s < p.T * kTopK;
  const int le = has_slot ? local_of(p.topk_ids[s], p.offset) : -1;
  const int rank = le >= 0 ? p.slot_rank[s] : 0;
  const float w = le >= 0 ? p.topk_w[s] : 0.f;
  // the token's local assignments (its 8 slots are 8 aligned lanes of this wavefront) decide
  // where GEMM2 sends the row: the token's output row if it has one, else its parked row
  const uint64_t lm = __ballot(le >= 0);
  const int tok = s / kTopK;
  const int dest = __popcll((lm >> (lane_id() & 56)) & 0xFFull) == 1 ? tok : -1 - s;

  if constexpr (SCANNED) {
    if (tid < kExpertsLocal) s_prefix[tid] = p.block_count[b * kExpertsLocal + tid];
    if (tid <= kExpertsLocal) s_start[tid] = p.expert_start[tid];
    __syncthreads();
    if (le < 0) return;
    const int pos = s_start[le] + s_prefix[le] + rank;
    p.sorted_token[pos] = tok;
    p.sorted_weight[pos] = w;
    p.sorted_slot[pos] = s;
    p.row_dest[pos] = dest;
    return;
  }
  const int e = tid % kExpertsLocal, j = tid / kExpertsLocal;
  int pre = 0, tot = 0;
  for (int b0 = j; b0 < nb; b0 += kPlaceGroups * kScanBatch) {
    int v[kScanBatch];
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) {
      const int bb = b0 + i * kPlaceGroups;
      v[i] = bb < nb ? p.block_count[bb * kExpertsLocal + e] : 0;
    }
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) {
      tot += v[i];
      pre += (b0 + i * kPlaceGroups < b) ? v[i] : 0;
    }
  }
  s_pre[j][e] = pre;
  s_tot[j][e] = tot;
  __syncthreads();
  if (tid < kExpertsLocal) {
    int pe = 0, te = 0;
#pragma unroll
    for (int jj = 0; jj < kPlaceGroups; ++jj) {
      pe += s_pre[jj][tid];
      te += s_tot[jj][tid];
    }
    s_prefix[tid] = pe;
    if (b == 0) {
      finish_counts(p, tid, te, s_start);
    } else {
      int incl = te;
#pragma unroll
      for (int off = 1; off < kExpertsLocal; off <<= 1) {
        const int o = __shfl_up(incl, off, kExpertsLocal);
        if (tid >= off) incl += o;
      }
      s_start[tid + 1] = incl;
      if (tid == 0) s_start[0] = 0;
    }
  }
  __syncthreads();
  if (le < 0) return;
  const int pos = s_start[le] + s_prefix[le] + rank;
  p.sorted_token[pos] = tok;
  p.sorted_weight[pos] = w;
  p.sorted_slot[pos] = s;
  p.row_dest[pos] = dest;
}

// Per-expert exclusive prefix of the routing work-groups' histograms, for batches of more than
// kPlaceDirectBlocks routing work-groups: one work-group of 1024 threads, thread (j, e) owning
// expert e's counts in the j-th of 32 contiguous ranges of work-groups. block_count is
// rewritten in place with the prefixes, and lanes 0..31 then write the CSR offsets, counters
// and work list (finish_counts) from the totals. O(work-groups) loads in all.
constexpr int kPlaceDirectBlocks = 1024;
constexpr int kBlockScanThreads = 1024;
constexpr int kBlockScanRanges = kBlockScanThreads / kExpertsLocal;   // 32

__global__ __launch_bounds__(kBlockScanThreads) void block_scan_kernel(RouteParams p) {
  __shared__ int s_sum[kBlockScanRanges][kExpertsLocal];
  __shared__ int s_start[kExpertsLocal + 1];
  const int tid = threadIdx.x;
  const int e = tid % kExpertsLocal, j = tid / kExpertsLocal;
  const int nb = p.nblocks;
  const int per = (nb + kBlockScanRanges - 1) / kBlockScanRanges;
  const int b0 = min(j * per, nb), b1 = min(b0 + per, nb);
  int sum = 0;
  for (int b = b0; b < b1; b += kScanBatch) {
    int v[kScanBatch];
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) v[i] = b + i < b1 ? p.block_count[(b + i) * kExpertsLocal + e] : 0;
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) sum += v[i];
  }
  s_sum[j][e] = sum;
  __syncthreads();
  int pre = 0, tot = 0;
#pragma unroll
  for (int jj = 0; jj < kBlockScanRanges; ++jj) {
    const int v = s_sum[jj][e];
    tot += v;
    pre += jj < j ? v : 0;
  }
  int run = pre;
  for (int b = b0; b < b1; b += kScanBatch) {
    int v[kScanBatch];
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i) v[i] = b + i < b1 ? p.block_count[(b + i) * kExpertsLocal + e] : 0;
#pragma unroll
    for (int i = 0; i < kScanBatch; ++i)
      if (b + i < b1) {
        p.block_count[(b + i) * kExpertsLocal + e] = run;
        run += v[i];
      }
  }
  if (tid < kExpertsLocal) finish_counts(p, tid, tot, s_start);
}

// top-k lists only (no dispatch), for batches of up to kWideRouteTokens tokens
static_assert(kWideRouteTokens >= kSinglePassTokens && kWideRouteTokens >= kFusedDispatchTokens,
              "every batch routed without ranks fits route_wide_kernel");
static hipError_t launch_route_lists(const RouteParams& p, hipStream_t s) {
  if (p.T > kWideRouteTokens) return hipErrorInvalidValue;
  hipLaunchKernelGGL(route_wide_kernel, dim3((p.T + 3) / 4), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_route(const RouteParams& p, hipStream_t s) { return launch_route_lists(p, s); }

hipError_t launch_route_dispatch(const RouteParams& p, hipStream_t s) {
  if (p.single_pass) {
    if (!p.skip_routing && launch_route_lists(p, s) != hipSuccess) return hipGetLastError();
    hipLaunchKernelGGL(dispatch_small_kernel, dim3(1), dim3(kRouteThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL(route_kernel, dim3(p.nblocks), dim3(kRouteWaves * 64), 0, s, p);
    if (p.nblocks > kPlaceDirectBlocks) {
      hipLaunchKernelGGL(block_scan_kernel, dim3(1), dim3(kBlockScanThreads), 0, s, p);
      hipLaunchKernelGGL(place_kernel<true>, dim3(p.nblocks), dim3(kPlaceThreads), 0, s, p);
    } else {
      hipLaunchKernelGGL(place_kernel<false>, dim3(p.nblocks), dim3(kPlaceThreads), 0, s, p);
    }
  }
  return hipGetLastError();
}

}  // namespace moe
