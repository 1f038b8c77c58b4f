// Grouped fp8 block-scale GEMMs of the MoE layer on gfx950 MFMA.
//
// Work item = (local expert e, a run of <= ROWS consecutive rows of e's bucket in the
// sorted assignment order). A work-group of 8 wavefronts takes one work item and one
// slice of output columns:
//   GEMM1: 128 SwiGLU columns -> 128 gate rows + 128 up rows of W13[e]; 16 column slices.
//   GEMM2: 256 hidden rows of W2[e]; 28 row slices.
// Each wavefront owns 32 weight rows (two 16-row MFMA fragments) and streams them from
// HBM straight into registers, NB K-steps ahead. The activation rows of the item (gathered
// by token for GEMM1, contiguous for GEMM2) are staged per 128-wide K-step in LDS
// (double buffered, XOR-swizzled 16-byte chunks) and shared by the 8 wavefronts.
// Every K-step is exactly one 128x128 scale block, so one v_mfma_f32_16x16x128_f8f6f4
// per fragment pair is followed by acc += mfma * (s_act[row,k] * s_w[block,k]) in fp32
// (kernel.py:123-124 and :234).
//
// Epilogues:
//   GEMM1: C = silu(X2) * X1 with X1 the first I columns and X2 the second (kernel.py:126-129),
//          then per row and 128 columns: scale = max(amax/448, 1e-12), q = e4m3(C/scale)
//          (kernel.py:131-135 uses 64-column blocks; this layer uses 128 so that GEMM2 sees
//          one activation scale per K-step).
//   GEMM2: v = acc * routing weight (kernel.py:236-237); a token with one local assignment
//          gets v written straight to its output row, others park v in `partial` by flat
//          slot for combine_kernel (the reference adds with fp32 atomics, kernel.py:246-250).
#include "moe_internal.h"
#include "moe_device.h"

namespace moe {

namespace {

constexpr int kG1 = 1;
constexpr int kG2 = 2;

template <int KIND>
struct GemmShape;
template <>
struct GemmShape<kG1> {
  static constexpr int kSteps = kHBlocks;        // K = 7168
  static constexpr int kRowBytes = kHidden;      // activation row stride
  static constexpr int kSlices = kG1ColBlocks;   // 16
};
template <>
struct GemmShape<kG2> {
  static constexpr int kSteps = kIBlocks;        // K = 2048
  static constexpr int kRowBytes = kInter;
  static constexpr int kSlices = kG2RowBlocks;   // 28
};

__device__ __forceinline__ int swz(int m, int c) { return m * 128 + ((c ^ (m & 7)) << 4); }

template <int KIND, int GROUPS, int NB>
__global__ __launch_bounds__(512) void gemm_kernel(GemmParams p) {
  using S = GemmShape<KIND>;
  constexpr int ROWS = GROUPS * 16;
  constexpr int KS = S::kSteps;
  constexpr int LITER = (ROWS * 8 + 511) / 512;  // 16-byte chunks per thread per K-step

  __shared__ __attribute__((aligned(16))) uint8_t s_tok[2][ROWS * 128];
  __shared__ float s_sa[2][ROWS];
  __shared__ float s_amax[kGemmWaves][ROWS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n_items = p.counters[kCtrItems];
  const int n_work = ((n_items + 7) & ~7) * S::kSlices;

  for (int w = blockIdx.x; w < n_work; w += gridDim.x) {
    // Work index -> (item, slice) keeping all slices of an item on one XCD (w % 8),
    // so the item's activation rows are fetched into one L2 only.
    const int xcd = w & 7, loc = w >> 3;
    const int slice = loc % S::kSlices;
    const int item = (loc / S::kSlices) * 8 + xcd;
    if (item >= n_items) continue;
    const int4 it = reinterpret_cast<const int4*>(p.work_items)[item];
    const int e = it.x, r0 = it.y, rows = it.z;
    const int ng = (rows + 15) >> 4;

    // ---- activation loader role: thread owns chunk (tid & 7) of rows (tid >> 3) + 64 i ----
    const uint8_t* a_src[LITER];
    bool a_ok[LITER];
#pragma unroll
    for (int i = 0; i < LITER; ++i) {
      const int m = (tid >> 3) + 64 * i;
      a_ok[i] = (m < rows) && (m < ROWS);
      size_t row = 0;
      if (a_ok[i]) {
        if constexpr (KIND == kG1) row = (size_t)p.sorted_token[r0 + m];
        else row = (size_t)(r0 + m);
      }
      const uint8_t* base = (KIND == kG1) ? p.hidden : p.act;
      a_src[i] = base + row * S::kRowBytes + (tid & 7) * 16;
    }
    const bool sa_ok = tid < rows && tid < ROWS;
    const float* sa_src = nullptr;
    if (sa_ok) {
      if constexpr (KIND == kG1) sa_src = p.hidden_scale + p.sorted_token[r0 + tid];  // + k*T
      else sa_src = p.act_scale + (size_t)(r0 + tid) * kIBlocks;                      // + k
    }
    auto load_a = [&](int k, v4i (&regs)[LITER], float& sa) {
#pragma unroll
      for (int i = 0; i < LITER; ++i)
        if (a_ok[i]) regs[i] = *reinterpret_cast<const v4i*>(a_src[i] + k * 128);
      if (sa_ok) {
        if constexpr (KIND == kG1) sa = sa_src[(size_t)k * p.T];
        else sa = sa_src[k];
      }
    };
    auto store_a = [&](int buf, const v4i (&regs)[LITER], float sa) {
#pragma unroll
      for (int i = 0; i < LITER; ++i) {
        const int m = (tid >> 3) + 64 * i;
        if (a_ok[i]) *reinterpret_cast<v4i*>(&s_tok[buf][swz(m, tid & 7)]) = regs[i];
      }
      if (sa_ok) s_sa[buf][tid] = sa;
    };

    // ---- weight rows of this wavefront ----
    const uint8_t* wf0;
    const uint8_t* wf1;
    const float* sw0;
    const float* sw1;
    if constexpr (KIND == kG1) {
      const int row = slice * kG1ColsPerBlock + wave * 16 + (lane & 15);   // gate row; up = +I
      wf0 = p.w13 + ((size_t)e * 2 * kInter + row) * kHidden + (lane >> 4) * 32;
      wf1 = wf0 + (size_t)kInter * kHidden;
      sw0 = p.w13_scale + ((size_t)e * 32 + slice) * kHBlocks;
      sw1 = p.w13_scale + ((size_t)e * 32 + kIBlocks + slice) * kHBlocks;
    } else {
      const int row = slice * kG2RowsPerBlock + wave * 32 + (lane & 15);
      wf0 = p.w2 + ((size_t)e * kHidden + row) * kInter + (lane >> 4) * 32;
      wf1 = wf0 + (size_t)16 * kInter;
      sw0 = p.w2_scale + ((size_t)e * kHBlocks + (slice * kG2RowsPerBlock + wave * 32) / 128) * kIBlocks;
      sw1 = sw0;
    }
    auto load_w = [&](int k, v8i (&dst)[2]) {
      const v4i* a = reinterpret_cast<const v4i*>(wf0 + k * 128);
      const v4i* b = reinterpret_cast<const v4i*>(wf1 + k * 128);
      dst[0] = join(a[0], a[1]);
      dst[1] = join(b[0], b[1]);
    };

    v8i wr[NB][2];
#pragma unroll
    for (int s = 0; s < NB - 1; ++s)
      if (s < KS) load_w(s, wr[s]);

    v4i areg[LITER];
    float sareg = 0.f;
    load_a(0, areg, sareg);
    store_a(0, areg, sareg);
    if (KS > 1) load_a(1, areg, sareg);
    __syncthreads();

    v4f acc0[GROUPS], acc1[GROUPS];
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
      acc0[g] = v4f{0.f, 0.f, 0.f, 0.f};
      acc1[g] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    const v4f zero = {0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < KS; k0 += NB) {
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int k = k0 + u;
        if (k < KS) {
          if (k + NB - 1 < KS) load_w(k + NB - 1, wr[(u + NB - 1) % NB]);
          if (k + 1 < KS) store_a((k + 1) & 1, areg, sareg);
          if (k + 2 < KS) load_a(k + 2, areg, sareg);
          const float s0 = sw0[k], s1 = sw1[k];
          const uint8_t* buf = s_tok[k & 1];
#pragma unroll
          for (int g = 0; g < GROUPS; ++g) {
            if (g < ng) {
              const int m = g * 16 + (lane & 15);
              const int c0 = (lane >> 4) * 2;
              const v8i bf = join(*reinterpret_cast<const v4i*>(&buf[swz(m, c0)]),
                                  *reinterpret_cast<const v4i*>(&buf[swz(m, c0 + 1)]));
              const float sa = s_sa[k & 1][m];
              const v4f d0 = mfma16x16x128_fp8(wr[u][0], bf, zero);
              const v4f d1 = mfma16x16x128_fp8(wr[u][1], bf, zero);
              const float f0 = sa * s0, f1 = sa * s1;
              acc0[g] += d0 * f0;
              acc1[g] += d1 * f1;
            }
          }
          __syncthreads();
        }
      }
    }

    // ---- epilogues ----
    if constexpr (KIND == kG1) {
      float c[GROUPS][4];
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) {
        if (g < ng) {
          float amax = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x1 = acc0[g][i], x2 = acc1[g][i];
            c[g][i] = (x2 / (1.0f + __expf(-x2))) * x1;
            amax = fmaxf(amax, fabsf(c[g][i]));
          }
          amax = fmaxf(amax, __shfl_xor(amax, 16));
          amax = fmaxf(amax, __shfl_xor(amax, 32));
          if (lane < 16) s_amax[wave][g * 16 + lane] = amax;
        }
      }
      __syncthreads();
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) {
        if (g < ng) {
          const int m = g * 16 + (lane & 15);
          float amax = s_amax[0][m];
#pragma unroll
          for (int ww = 1; ww < kGemmWaves; ++ww) amax = fmaxf(amax, s_amax[ww][m]);
          const float scale = fmaxf(amax / 448.0f, 1e-12f);
          if (m < rows) {
            const uint32_t q = pack_fp8x4(c[g][0] / scale, c[g][1] / scale, c[g][2] / scale,
                                          c[g][3] / scale);
            const int col = slice * kG1ColsPerBlock + wave * 16 + 4 * (lane >> 4);
            *reinterpret_cast<uint32_t*>(p.act + (size_t)(r0 + m) * kInter + col) = q;
            if (wave == 0 && lane < 16) p.act_scale[(size_t)(r0 + m) * kIBlocks + slice] = scale;
          }
        }
      }
      __syncthreads();
    } else {
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) {
        if (g < ng) {
          const int m = g * 16 + (lane & 15);
          if (m < rows) {
            const int pr = r0 + m;
            const int t = p.sorted_token[pr];
            const float wt = p.sorted_weight[pr];
            const bool direct = p.token_nlocal[t] == 1;
            const size_t slot = (size_t)p.sorted_slot[pr];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
              const v4f v = (f == 0 ? acc0[g] : acc1[g]) * wt;
              const int h = slice * kG2RowsPerBlock + wave * 32 + f * 16 + 4 * (lane >> 4);
              if (direct) {
                if (p.out_dtype == MOE_FP8_OUT_BF16) {
                  *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + (size_t)t * kHidden + h) =
                      pack_bf16x4(v[0], v[1], v[2], v[3]);
                } else {
                  *reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.out) + (size_t)t * kHidden + h) = v;
                }
              } else {
                *reinterpret_cast<v4f*>(p.partial + slot * kHidden + h) = v;
              }
            }
          }
        }
      }
    }
  }
}

// Sums the parked GEMM2 rows of every token without exactly one local assignment, in
// top-k slot order, and writes its output row (zeros for a token with none).
__global__ __launch_bounds__(256) void combine_kernel(GemmParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int t = blockIdx.x * 4 + wave; t < p.T; t += gridDim.x * 4) {
    if (p.token_nlocal[t] == 1) continue;
    unsigned local_mask = 0;
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
      const int le = p.topk_ids[t * kTopK + k] - p.offset;
      if (le >= 0 && le < kExpertsLocal) local_mask |= 1u << k;
    }
    const v4f* rows = reinterpret_cast<const v4f*>(p.partial + (size_t)t * kTopK * kHidden);
    for (int h4 = lane; h4 < kHidden / 4; h4 += 64) {
      v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < kTopK; ++k)
        if ((local_mask >> k) & 1u) acc += rows[(size_t)k * (kHidden / 4) + h4];
      if (p.out_dtype == MOE_FP8_OUT_BF16)
        reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + (size_t)t * kHidden)[h4] =
            pack_bf16x4(acc[0], acc[1], acc[2], acc[3]);
      else
        reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.out) + (size_t)t * kHidden)[h4] = acc;
    }
  }
}

int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int KIND, int GROUPS>
hipError_t launch_kind(const GemmParams& p, hipStream_t s) {
  using S = GemmShape<KIND>;
  const int max_work = ((p.max_items + 7) & ~7) * S::kSlices;
  int grid = num_cus() * 2;
  grid = (grid + 7) & ~7;
  if (grid > max_work) grid = max_work;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_kernel<KIND, GROUPS, 4>), dim3(grid), dim3(512), 0, s, p);
  return hipGetLastError();
}

template <int KIND>
hipError_t launch_rows(const GemmParams& p, int rows_per_item, hipStream_t s) {
  switch (rows_per_item) {
    case 16: return launch_kind<KIND, 1>(p, s);
    case 32: return launch_kind<KIND, 2>(p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gemm1(const GemmParams& p, int rows_per_item, hipStream_t s) {
  return launch_rows<kG1>(p, rows_per_item, s);
}

hipError_t launch_gemm2(const GemmParams& p, int rows_per_item, hipStream_t s) {
  return launch_rows<kG2>(p, rows_per_item, s);
}

hipError_t launch_combine(const GemmParams& p, hipStream_t s) {
  if (p.T <= 0) return hipSuccess;
  int grid = (p.T + 3) / 4;
  if (grid > 2048) grid = 2048;
  hipLaunchKernelGGL(combine_kernel, dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace moe
