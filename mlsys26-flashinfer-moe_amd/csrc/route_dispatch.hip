// Routing and dispatch for the fused MoE layer (gfx950).
//
// route_dispatch_kernel: one wavefront per token computes the DeepSeek-V3 no-aux grouped
// routing (kernel.py:428-542), then the work-group of 16 tokens builds its slice of the
// expert histogram together with the stable rank of each local assignment inside the
// work-group. The last work-group to finish (ticket counter) scans the per-work-group
// histograms into CSR offsets, builds the GEMM work list and, for small T, places every
// assignment itself. place_kernel places the assignments for larger T.
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

// (value, index) order used by every argmax of the routing: larger value first, then
// lower index (the "lowest index on ties" rule of kernel.py:499 and :525).
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Routes token t with the calling wavefront. Lane l owns global experts 4l..4l+3.
// On return every lane holds the 8 selected expert ids and weights in selection order.
__device__ void route_token(const RouteParams& p, int t, int (&ids)[kTopK], float (&wts)[kTopK]) {
  const int lane = lane_id();
  const float4 lg = reinterpret_cast<const float4*>(p.logits + (size_t)t * kExpertsGlobal)[lane];
  const float lgv[4] = {lg.x, lg.y, lg.z, lg.w};
  float s[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = sigmoid_f32(lgv[i]);                                   // kernel.py:466
    b[i] = s[i] + load_bias(p.bias, p.bias_dtype, 4 * lane + i);  // kernel.py:467
  }
  // Group score = sum of the two largest biased scores of the group (kernel.py:479-488).
  // The 32 experts of group g live in lanes 8g..8g+7.
  float m1 = fmaxf(b[0], b[1]), m2 = fminf(b[0], b[1]);
  top2_merge(m1, m2, fmaxf(b[2], b[3]), fminf(b[2], b[3]));
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    const float o1 = __shfl_xor(m1, off);
    const float o2 = __shfl_xor(m2, off);
    top2_merge(m1, m2, o1, o2);
  }
  const float my_group_score = m1 + m2;
  float gs[kNGroup];
#pragma unroll
  for (int g = 0; g < kNGroup; ++g) gs[g] = __shfl(my_group_score, g * 8);

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
    float bv = v[0];
    int bi = 4 * lane;
#pragma unroll
    for (int i = 1; i < 4; ++i)
      if (v[i] > bv) { bv = v[i]; bi = 4 * lane + i; }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int owner = bi >> 2, sub = bi & 3;
    const float my_s = sub == 0 ? s[0] : sub == 1 ? s[1] : sub == 2 ? s[2] : s[3];
    wts[k] = __shfl(my_s, owner);
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

// Writes the sorted entries of flat slot s (token s/8) if it is local.
__device__ __forceinline__ void place_slot(const RouteParams& p, int s, const int* start,
                                           const int32_t* block_base) {
  const int le = local_of(p.topk_ids[s], p.offset);
  if (le < 0) return;
  const int blk = s / (kRouteTokensPerBlock * kTopK);
  const int pos = start[le] + block_base[blk * kExpertsLocal + le] + p.slot_rank[s];
  p.sorted_token[pos] = s / kTopK;
  p.sorted_weight[pos] = p.topk_w[s];
  p.sorted_slot[pos] = s;
}

}  // namespace

__global__ __launch_bounds__(kRouteThreads) void route_dispatch_kernel(RouteParams p) {
  __shared__ int s_le[kRouteTokensPerBlock * kTopK];
  __shared__ int s_wcnt[2][kExpertsLocal];
  __shared__ int s_part[32][kExpertsLocal];
  __shared__ int s_start[kExpertsLocal + 1];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int t = blockIdx.x * kRouteTokensPerBlock + wave;

  // ---- routing (or reuse of given top-k lists) ----
  int my_id = -1;
  if (t < p.T) {
    if (!p.skip_routing) {
      int ids[kTopK];
      float wts[kTopK];
      route_token(p, t, ids, wts);
      int id_k = 0;
      float w_k = 0.f;
#pragma unroll
      for (int k = 0; k < kTopK; ++k)
        if (lane == k) { id_k = ids[k]; w_k = wts[k]; }
      if (lane < kTopK) {
        p.topk_ids[t * kTopK + lane] = id_k;
        p.topk_w[t * kTopK + lane] = w_k;
        my_id = id_k;
      }
    } else if (lane < kTopK) {
      my_id = p.topk_ids[t * kTopK + lane];
    }
  }
  const int le = (t < p.T && lane < kTopK) ? local_of(my_id, p.offset) : -1;
  const uint64_t local_mask = __ballot(le >= 0);
  if (lane < kTopK) s_le[wave * kTopK + lane] = le;
  if (lane == 0 && t < p.T) p.token_nlocal[t] = __popcll(local_mask);
  __syncthreads();

  // ---- work-group histogram and stable rank of each local slot ----
  const int slot0 = blockIdx.x * kRouteTokensPerBlock * kTopK;
  const int nslots = p.T * kTopK;
  int my_le = -1, rank = 0, cnt = 0;
  if (tid < kRouteTokensPerBlock * kTopK) {
    my_le = s_le[tid];
    const uint64_t lt = lanemask_lt();
#pragma unroll 4
    for (int e = 0; e < kExpertsLocal; ++e) {
      const uint64_t m = __ballot(my_le == e);
      if (my_le == e) rank = __popcll(m & lt);
      if (lane == e) cnt = __popcll(m);
    }
    if (lane < kExpertsLocal) s_wcnt[wave][lane] = cnt;
  }
  __syncthreads();
  if (tid < kRouteTokensPerBlock * kTopK) {
    if (my_le >= 0 && slot0 + tid < nslots) {
      if (wave == 1) rank += s_wcnt[0][my_le];
      p.slot_rank[slot0 + tid] = rank;
    }
    if (tid < kExpertsLocal)
      p.block_count[blockIdx.x * kExpertsLocal + tid] = s_wcnt[0][tid] + s_wcnt[1][tid];
  }

  // ---- the last work-group scans ----
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = (atomicAdd(&p.counters[kCtrTicket], 1) == p.nblocks - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const int nb = p.nblocks;
  {
    const int e = tid & 31, j = tid >> 5;  // 32 threads per expert
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
      // expert totals and CSR offsets (kernel.py:357-360)
      int incl = run;
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) {
        const int o = __shfl_up(incl, off, 32);
        if (tid >= off) incl += o;
      }
      p.expert_count[tid] = run;
      p.expert_start[tid + 1] = incl;
      s_start[tid + 1] = incl;
      if (tid == 0) { p.expert_start[0] = 0; s_start[0] = 0; }
      if (tid == kExpertsLocal - 1) p.counters[kCtrAssign] = incl;
      // GEMM work list: each expert's rows cut into items of rows_per_item rows
      // (kernel.py:384-407 builds the equivalent per-tile table).
      const int bm = p.rows_per_item;
      const int nch = (run + bm - 1) / bm;
      int ich = nch;
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) {
        const int o = __shfl_up(ich, off, 32);
        if (tid >= off) ich += o;
      }
      const int first = ich - nch;
      const int start = incl - run;
      for (int c = 0; c < nch; ++c) {
        int4 it;
        it.x = tid;
        it.y = start + c * bm;
        it.z = min(bm, run - c * bm);
        it.w = 0;
        reinterpret_cast<int4*>(p.work_items)[first + c] = it;
      }
      if (tid == kExpertsLocal - 1) p.counters[kCtrItems] = ich;
      if (tid == 0) p.counters[kCtrTicket] = 0;
    }
    __syncthreads();
    int run = s_part[j][e];
    for (int b = b0; b < b1; ++b) {
      const int v = p.block_count[b * kExpertsLocal + e];
      p.block_count[b * kExpertsLocal + e] = run;
      run += v;
    }
  }
  if (!p.single_pass) return;
  // The prefixes just written to block_count are re-read through the vector L1 below.
  __threadfence();
  __syncthreads();
  for (int s = tid; s < nslots; s += kRouteThreads) place_slot(p, s, s_start, p.block_count);
}

__global__ __launch_bounds__(kRouteTokensPerBlock * kTopK) void place_kernel(RouteParams p) {
  __shared__ int s_start[kExpertsLocal + 1];
  if (threadIdx.x <= kExpertsLocal) s_start[threadIdx.x] = p.expert_start[threadIdx.x];
  __syncthreads();
  const int s = blockIdx.x * kRouteTokensPerBlock * kTopK + threadIdx.x;
  if (s < p.T * kTopK) place_slot(p, s, s_start, p.block_count);
}

hipError_t launch_route_dispatch(const RouteParams& p, hipStream_t s) {
  hipLaunchKernelGGL(route_dispatch_kernel, dim3(p.nblocks), dim3(kRouteThreads), 0, s, p);
  if (!p.single_pass)
    hipLaunchKernelGGL(place_kernel, dim3(p.nblocks), dim3(kRouteTokensPerBlock * kTopK), 0, s, p);
  return hipGetLastError();
}

}  // namespace moe
