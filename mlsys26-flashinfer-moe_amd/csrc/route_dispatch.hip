// Routing and dispatch for the fused MoE layer (gfx950).
//
// One wavefront per token computes the DeepSeek-V3 no-aux grouped routing (kernel.py:428-542)
// with DPP/readlane reductions. Dispatch then histograms the local assignments, scans them
// into CSR offsets, builds the GEMM work list and places every assignment in its bucket:
//   T <= 256: route_dispatch_small_kernel does everything in one work-group, in LDS;
//   larger T: route_count_kernel (per work-group histograms and ranks) -> scan_kernel ->
//             place_kernel. No kernel synchronises across work-groups.
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

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

// Argmax key of the routing: a larger fp32 value wins, then the lower index (the "lowest
// index on ties" rule of kernel.py:499 and :525). The value is mapped to an unsigned key
// that orders like the float (after -0 -> +0, so that equal values tie).
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  uint32_t u = __float_as_uint(v + 0.0f);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)(0xFFFF - idx);
}

__device__ __forceinline__ int key_index(uint64_t key) { return 0xFFFF - (int)(key & 0xFFFFu); }

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Wave-wide maximum of a key, returned uniformly: DPP inside each 16-lane row, then the
// four row results combined through readlane.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
  k = max_u64(k, dpp_u64<kDppXor1>(k));
  k = max_u64(k, dpp_u64<kDppXor2>(k));
  k = max_u64(k, dpp_u64<kDppHalfMirror>(k));
  k = max_u64(k, dpp_u64<kDppMirror>(k));
  const uint64_t r0 = readlane_u64(k, 0), r1 = readlane_u64(k, 16);
  const uint64_t r2 = readlane_u64(k, 32), r3 = readlane_u64(k, 48);
  return max_u64(max_u64(r0, r1), max_u64(r2, r3));
}

// Routes token t with the calling wavefront. Lane l owns global experts 4l..4l+3.
// On return every lane holds the 8 selected expert ids and weights in selection order.
__device__ void route_token(const RouteParams& p, const float* s_bias, int t, int (&ids)[kTopK],
                            float (&wts)[kTopK]) {
  const int lane = lane_id();
  const float4 lg = reinterpret_cast<const float4*>(p.logits + (size_t)t * kExpertsGlobal)[lane];
  const float4 bs = reinterpret_cast<const float4*>(s_bias)[lane];
  const float lgv[4] = {lg.x, lg.y, lg.z, lg.w};
  const float bv[4] = {bs.x, bs.y, bs.z, bs.w};
  float s[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = sigmoid_f32(lgv[i]);   // kernel.py:466
    b[i] = s[i] + bv[i];          // kernel.py:467
  }
  // Group score = sum of the two largest biased scores of the group (kernel.py:479-488).
  // The 32 experts of group g live in lanes 8g..8g+7.
  float m1 = fmaxf(b[0], b[1]), m2 = fminf(b[0], b[1]);
  top2_merge(m1, m2, fmaxf(b[2], b[3]), fminf(b[2], b[3]));
  top2_merge(m1, m2, dpp_f32<kDppXor1>(m1), dpp_f32<kDppXor1>(m2));
  top2_merge(m1, m2, dpp_f32<kDppXor2>(m1), dpp_f32<kDppXor2>(m2));
  top2_merge(m1, m2, dpp_f32<kDppHalfMirror>(m1), dpp_f32<kDppHalfMirror>(m2));
  const float my_group_score = m1 + m2;
  float gs[kNGroup];
#pragma unroll
  for (int g = 0; g < kNGroup; ++g)
    gs[g] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_group_score), g * 8));

  // Keep the top-4 groups: 4 rounds of max over the unselected groups, lowest index on
  // ties (kernel.py:495-501).
  int selected = 0;
#pragma unroll
  for (int r = 0; r < kTopKGroup; ++r) {
    float best = -INFINITY;
#pragma unroll
    for (int g = 0; g < kNGroup; ++g) {
      const float v = ((selected >> g) & 1) ? -INFINITY : gs[g];
      best = fmaxf(best, v);
    }
    int bg = kNGroup;
#pragma unroll
    for (int g = kNGroup - 1; g >= 0; --g) {
      const float v = ((selected >> g) & 1) ? -INFINITY : gs[g];
      if (!((selected >> g) & 1) && v == best) bg = g;
    }
    if (bg < kNGroup) selected |= 1 << bg;
  }

  // Top-8 experts of the kept groups by biased score, lowest index on ties; the weight
  // uses the unbiased score (kernel.py:515-534).
  const bool mine = (selected >> (lane >> 3)) & 1;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = mine ? b[i] : -INFINITY;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    uint64_t best = argmax_key(v[0], 4 * lane);
#pragma unroll
    for (int i = 1; i < 4; ++i) best = max_u64(best, argmax_key(v[i], 4 * lane + i));
    const int bi = key_index(wave_max_key(best));
    const int owner = bi >> 2, sub = bi & 3;
    const float my_s = sub == 0 ? s[0] : sub == 1 ? s[1] : sub == 2 ? s[2] : s[3];
    wts[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_s), owner));
    ids[k] = bi;
    if (lane == owner) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i == sub) v[i] = -INFINITY;
    }
  }
  // Renormalise and scale: w = s / (sum s + 1e-20) * rsf, sum taken in selection order
  // (kernel.py:537-538).
  float sum = wts[0];
#pragma unroll
  for (int k = 1; k < kTopK; ++k) sum = sum + wts[k];
  sum = sum + 1e-20f;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) wts[k] = __fdiv_rn(wts[k], sum) * p.rsf;
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

// Routes token t with the calling wavefront (or reads its given top-k list) and stores the
// result; returns, in lanes 0..7, the local expert index of slot t*8+lane (-1 if not local)
// and its routing weight.
__device__ __forceinline__ int route_or_load(const RouteParams& p, const float* s_bias, int t, float& w_out) {
  const int lane = lane_id();
  int id = -1;
  float w = 0.f;
  if (!p.skip_routing) {
    int ids[kTopK];
    float wts[kTopK];
    route_token(p, s_bias, t, ids, wts);
#pragma unroll
    for (int k = 0; k < kTopK; ++k)
      if (lane == k) { id = ids[k]; w = wts[k]; }
    if (lane < kTopK) {
      p.topk_ids[t * kTopK + lane] = id;
      p.topk_w[t * kTopK + lane] = w;
    }
  } else if (lane < kTopK) {
    id = p.topk_ids[t * kTopK + lane];
    w = p.topk_w[t * kTopK + lane];
  }
  const int le = lane < kTopK ? local_of(id, p.offset) : -1;
  const uint64_t local_mask = __ballot(le >= 0);
  if (lane == 0) p.token_nlocal[t] = __popcll(local_mask);
  w_out = w;
  return le;
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
}

}  // namespace

// Small batches (T <= kSinglePassTokens): routing and the whole dispatch in one work-group.
// Each wavefront routes tokens wave, wave+16, ...; the local expert ids and weights of all
// T*8 slots stay in LDS, are ranked 1024 at a time and placed without leaving the
// work-group, so no cross-work-group synchronisation is needed.
__global__ __launch_bounds__(kRouteThreads) void route_dispatch_small_kernel(RouteParams p) {
  __shared__ __attribute__((aligned(16))) float s_bias[kExpertsGlobal];
  __shared__ int s_le[kSinglePassTokens * kTopK];
  __shared__ int s_rank[kSinglePassTokens * kTopK];
  __shared__ float s_w[kSinglePassTokens * kTopK];
  __shared__ int s_wcnt[16][kExpertsLocal];
  __shared__ int s_cnt[kExpertsLocal];
  __shared__ int s_base[kExpertsLocal];
  __shared__ int s_start[kExpertsLocal + 1];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int nslots = p.T * kTopK;
  stage_bias(p, s_bias);
  for (int t = wave; t < p.T; t += kRouteTokensPerBlock) {
    float w;
    const int le = route_or_load(p, s_bias, t, w);
    if (lane < kTopK) {
      s_le[t * kTopK + lane] = le;
      s_w[t * kTopK + lane] = w;
    }
  }
  if (tid < kExpertsLocal) s_base[tid] = 0;
  __syncthreads();
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

// Large batches, step 1: one wavefront per token; the work-group of 16 tokens records each
// local slot's stable rank inside the work-group and the work-group's expert histogram.
__global__ __launch_bounds__(kRouteThreads) void route_count_kernel(RouteParams p) {
  __shared__ __attribute__((aligned(16))) float s_bias[kExpertsGlobal];
  __shared__ int s_le[kRouteTokensPerBlock * kTopK];
  __shared__ int s_wcnt[16][kExpertsLocal];
  __shared__ int s_cnt[kExpertsLocal];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int t = blockIdx.x * kRouteTokensPerBlock + wave;
  stage_bias(p, s_bias);
  int le = -1;
  if (t < p.T) {
    float w;
    le = route_or_load(p, s_bias, t, w);
  }
  if (lane < kTopK) s_le[wave * kTopK + lane] = le;
  __syncthreads();
  // the 128 slots of the work-group are held by threads 0..127 (wavefronts 0 and 1)
  const int my_le = tid < kRouteTokensPerBlock * kTopK ? s_le[tid] : -1;
  const int r = block_rank(my_le, kRouteThreads / 64, s_wcnt, s_cnt);
  const int slot = blockIdx.x * kRouteTokensPerBlock * kTopK + tid;
  if (my_le >= 0) p.slot_rank[slot] = r;
  if (tid < kExpertsLocal) p.block_count[blockIdx.x * kExpertsLocal + tid] = s_cnt[tid];
}

// Large batches, step 2 (one work-group): per-expert exclusive prefix of the work-group
// histograms (in place), CSR offsets and the work list.
__global__ __launch_bounds__(kRouteThreads) void scan_kernel(RouteParams p) {
  __shared__ int s_part[32][kExpertsLocal];
  __shared__ int s_start[kExpertsLocal + 1];
  const int tid = threadIdx.x;
  const int nb = p.nblocks;
  const int e = tid & 31, j = tid >> 5;   // 32 threads per expert
  const int chunk = (nb + 31) / 32;
  const int b0 = min(nb, j * chunk), b1 = min(nb, b0 + chunk);
  int sum = 0;
  for (int b = b0; b < b1; ++b) sum += p.block_count[b * kExpertsLocal + e];
  s_part[j][e] = sum;
  __syncthreads();
  if (tid < kExpertsLocal) {
    int run = 0;
    for (int jj = 0; jj < 32; ++jj) {
      const int v = s_part[jj][tid];
      s_part[jj][tid] = run;
      run += v;
    }
    finish_counts(p, tid, run, s_start);
  }
  __syncthreads();
  int run = s_part[j][e];
  for (int b = b0; b < b1; ++b) {
    const int v = p.block_count[b * kExpertsLocal + e];
    p.block_count[b * kExpertsLocal + e] = run;
    run += v;
  }
}

// Large batches, step 3: each local slot to its bucket position.
__global__ __launch_bounds__(kRouteTokensPerBlock * kTopK) void place_kernel(RouteParams p) {
  __shared__ int s_start[kExpertsLocal + 1];
  if (threadIdx.x <= kExpertsLocal) s_start[threadIdx.x] = p.expert_start[threadIdx.x];
  __syncthreads();
  const int s = blockIdx.x * kRouteTokensPerBlock * kTopK + threadIdx.x;
  if (s >= p.T * kTopK) return;
  const int le = local_of(p.topk_ids[s], p.offset);
  if (le < 0) return;
  const int pos = s_start[le] + p.block_count[blockIdx.x * kExpertsLocal + le] + p.slot_rank[s];
  p.sorted_token[pos] = s / kTopK;
  p.sorted_weight[pos] = p.topk_w[s];
  p.sorted_slot[pos] = s;
}

hipError_t launch_route_dispatch(const RouteParams& p, hipStream_t s) {
  if (p.single_pass) {
    hipLaunchKernelGGL(route_dispatch_small_kernel, dim3(1), dim3(kRouteThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL(route_count_kernel, dim3(p.nblocks), dim3(kRouteThreads), 0, s, p);
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(kRouteThreads), 0, s, p);
    hipLaunchKernelGGL(place_kernel, dim3(p.nblocks), dim3(kRouteTokensPerBlock * kTopK), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace moe
