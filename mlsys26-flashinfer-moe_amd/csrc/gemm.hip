// Grouped fp8 block-scale GEMMs of the MoE layer on gfx950 MFMA.
//
// Work item = (local expert e, a run of <= ROWS consecutive rows of e's bucket in the
// sorted assignment order). A work-group of 8 wavefronts takes one work item and one
// slice of output columns:
//   GEMM1: 128 SwiGLU columns -> 128 gate rows + 128 up rows of W13[e]; 16 column slices.
//   GEMM2: 256 hidden rows of W2[e]; 28 row slices.
// Each wavefront owns 32 weight rows (two 16-row MFMA fragments) and streams them from
// HBM straight into registers, several K-steps ahead. Every K-step is exactly one 128x128
// scale block, so one v_mfma_f32_16x16x128_f8f6f4 per fragment pair is followed by
// acc += mfma * (s_act[row,k] * s_w[block,k]) in fp32 (kernel.py:123-124 and :234).
//
// gemm_stream_kernel serves items of <= 32 rows (the decode regime): each wavefront also
// loads the activation fragments of the item itself, into the same in-order register ring
// as its weights; there is no LDS traffic and no barrier in the K loop. Items of up to 128
// rows go to the tile kernels of gemm_tile.hip.
//
// K-byte permutation: inside each 128-byte K block, lane group g = lane/16 holds bytes
// [16g, 16g+16) and [64+16g, 64+16g+16) of its row (weights and activations alike, so the
// dot products are unchanged). Each 16-byte load instruction of a wavefront then reads
// whole 64-byte segments of 16 rows.
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

// One MFMA operand fragment: bytes [16g, 16g+16) and [64+16g, +16) of a 128-byte K block
// (p already points at row + 16g).
__device__ __forceinline__ v8i load_frag(const uint8_t* p) {
  const v4i lo = *reinterpret_cast<const v4i*>(p);
  const v4i hi = *reinterpret_cast<const v4i*>(p + 64);
  return join(lo, hi);
}

// Decodes work index w into (item, slice): all slices of an item stay on one XCD (w % 8),
// so the item's activation rows are fetched into one L2.
template <int SLICES>
__device__ __forceinline__ bool decode_work(int w, int n_items, int& item, int& slice) {
  const int xcd = w & 7, loc = w >> 3;
  slice = loc % SLICES;
  item = (loc / SLICES) * 8 + xcd;
  return item < n_items;
}

// Weight fragment rows and block-scale rows of this wavefront.
template <int KIND>
__device__ __forceinline__ void weight_rows(const GemmParams& p, int e, int slice, int wave, int lane,
                                            const uint8_t*& wf0, const uint8_t*& wf1, const float*& sw0,
                                            const float*& sw1) {
  if constexpr (KIND == kG1) {
    const int row = slice * kG1ColsPerBlock + wave * 16 + (lane & 15);   // gate row; up = +I
    wf0 = p.w13 + ((size_t)e * 2 * kInter + row) * kHidden + (lane >> 4) * 16;
    wf1 = wf0 + (size_t)kInter * kHidden;
    sw0 = p.w13_scale + ((size_t)e * 32 + slice) * kHBlocks;
    sw1 = p.w13_scale + ((size_t)e * 32 + kIBlocks + slice) * kHBlocks;
  } else {
    const int row = slice * kG2RowsPerBlock + wave * 32 + (lane & 15);
    wf0 = p.w2 + ((size_t)e * kHidden + row) * kInter + (lane >> 4) * 16;
    wf1 = wf0 + (size_t)16 * kInter;
    sw0 = p.w2_scale + ((size_t)e * kHBlocks + (slice * kG2RowsPerBlock + wave * 32) / 128) * kIBlocks;
    sw1 = sw0;
  }
}

// GEMM1 epilogue: SwiGLU, row amax over the work-group's 128 columns, fp8 requantisation.
template <int GROUPS>
__device__ __forceinline__ void epilogue_gemm1(const GemmParams& p, const v4f (&acc0)[GROUPS],
                                               const v4f (&acc1)[GROUPS], int ng, int rows, int r0,
                                               int slice, int wave, int lane,
                                               float (*s_amax)[GROUPS * 16]) {
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
        const uint32_t q = pack_fp8x4(c[g][0] / scale, c[g][1] / scale, c[g][2] / scale, c[g][3] / scale);
        const int col = slice * kG1ColsPerBlock + wave * 16 + 4 * (lane >> 4);
        *reinterpret_cast<uint32_t*>(p.act + (size_t)(r0 + m) * kInter + col) = q;
        if (wave == 0 && lane < 16) p.act_scale[(size_t)(r0 + m) * kIBlocks + slice] = scale;
      }
    }
  }
  __syncthreads();
}

// GEMM2 epilogue: weight by the routing weight; single-assignment tokens write their output
// row directly, the others park the row in `partial` under its flat slot.
template <int GROUPS>
__device__ __forceinline__ void epilogue_gemm2(const GemmParams& p, const v4f (&acc0)[GROUPS],
                                               const v4f (&acc1)[GROUPS], int ng, int rows, int r0,
                                               int slice, int wave, int lane) {
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

template <int GROUPS>
struct StreamStage {
  v8i w[2];
  v8i a[GROUPS];
  float sa[GROUPS];
  float sw[2];
};

template <int KIND, int GROUPS, int NB>
__global__ __launch_bounds__(512) void gemm_stream_kernel(GemmParams p) {
  using S = GemmShape<KIND>;
  constexpr int KS = S::kSteps;
  __shared__ float s_amax[kGemmWaves][GROUPS * 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n_items = min(p.counters[kCtrItems], p.max_items);
  const int n_work = ((n_items + 7) & ~7) * S::kSlices;

  for (int w = blockIdx.x; w < n_work; w += gridDim.x) {
    int item, slice;
    if (!decode_work<S::kSlices>(w, n_items, item, slice)) continue;
    const int4 it = reinterpret_cast<const int4*>(p.work_items)[item];
    const int e = it.x, r0 = it.y, rows = it.z;
    const int ng = (rows + 15) >> 4;

    const uint8_t *wf0, *wf1;
    const float *sw0, *sw1;
    weight_rows<KIND>(p, e, slice, wave, lane, wf0, wf1, sw0, sw1);

    // Activation rows of this lane's column in each 16-row group (rows past the item's end
    // read its first row; their results are never stored).
    const uint8_t* ap[GROUPS];
    const float* sap[GROUPS];
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
      const int m = g * 16 + (lane & 15);
      const int mm = m < rows ? m : 0;
      if constexpr (KIND == kG1) {
        const int tok = p.sorted_token[r0 + mm];
        ap[g] = p.hidden + (size_t)tok * kHidden + (lane >> 4) * 16;
        sap[g] = p.hidden_scale + tok;
      } else {
        ap[g] = p.act + (size_t)(r0 + mm) * kInter + (lane >> 4) * 16;
        sap[g] = p.act_scale + (size_t)(r0 + mm) * kIBlocks;
      }
    }
    const size_t sa_stride = (KIND == kG1) ? (size_t)p.T : 1;

    StreamStage<GROUPS> ring[NB];
    auto issue = [&](int k, StreamStage<GROUPS>& st) {
      st.w[0] = load_frag(wf0 + k * 128);
      st.w[1] = load_frag(wf1 + k * 128);
#pragma unroll
      for (int g = 0; g < GROUPS; ++g) {
        if (g < ng) {
          st.a[g] = load_frag(ap[g] + k * 128);
          st.sa[g] = sap[g][k * sa_stride];
        }
      }
      st.sw[0] = sw0[k];
      st.sw[1] = sw1[k];
    };
#pragma unroll
    for (int s = 0; s < NB - 1; ++s)
      if (s < KS) issue(s, ring[s]);

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
          if (k + NB - 1 < KS) issue(k + NB - 1, ring[(u + NB - 1) % NB]);
          const StreamStage<GROUPS>& st = ring[u];
#pragma unroll
          for (int g = 0; g < GROUPS; ++g) {
            if (g < ng) {
              const v4f d0 = mfma16x16x128_fp8(st.w[0], st.a[g], zero);
              const v4f d1 = mfma16x16x128_fp8(st.w[1], st.a[g], zero);
              acc0[g] += d0 * (st.sa[g] * st.sw[0]);
              acc1[g] += d1 * (st.sa[g] * st.sw[1]);
            }
          }
        }
      }
    }
    if constexpr (KIND == kG1) epilogue_gemm1<GROUPS>(p, acc0, acc1, ng, rows, r0, slice, wave, lane, s_amax);
    else epilogue_gemm2<GROUPS>(p, acc0, acc1, ng, rows, r0, slice, wave, lane);
  }
}

// Output rows of every token without exactly one local assignment: the sum of its parked
// GEMM2 rows in top-k slot order, or zeros. One thread per 4 columns of one token row.
__global__ __launch_bounds__(256) void combine_kernel(GemmParams p) {
  constexpr int kVecPerRow = kHidden / 4;   // 1792
  const size_t total = (size_t)p.T * kVecPerRow;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(i / kVecPerRow);
    const int h4 = (int)(i - (size_t)t * kVecPerRow);
    if (p.token_nlocal[t] == 1) continue;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    const v4f* rows = reinterpret_cast<const v4f*>(p.partial + (size_t)t * kTopK * kHidden);
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
      const int le = p.topk_ids[t * kTopK + k] - p.offset;
      if (le >= 0 && le < kExpertsLocal) acc += rows[(size_t)k * kVecPerRow + h4];
    }
    if (p.out_dtype == MOE_FP8_OUT_BF16)
      reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + (size_t)t * kHidden)[h4] =
          pack_bf16x4(acc[0], acc[1], acc[2], acc[3]);
    else
      reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.out) + (size_t)t * kHidden)[h4] = acc;
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

int persistent_grid(int max_work, int blocks_per_cu) {
  int grid = num_cus() * blocks_per_cu;
  grid = (grid + 7) & ~7;
  return grid < max_work ? grid : max_work;
}

template <int KIND>
hipError_t launch_rows(const GemmParams& p, int rows_per_item, hipStream_t s) {
  using S = GemmShape<KIND>;
  const int max_work = ((p.max_items + 7) & ~7) * S::kSlices;
  switch (rows_per_item) {
    case 16: {
      const int grid = persistent_grid(max_work, 2);
      if (grid > 0) hipLaunchKernelGGL((gemm_stream_kernel<KIND, 1, 3>), dim3(grid), dim3(512), 0, s, p);
      break;
    }
    case 32: {
      const int grid = persistent_grid(max_work, 1);
      if (grid > 0) hipLaunchKernelGGL((gemm_stream_kernel<KIND, 2, 3>), dim3(grid), dim3(512), 0, s, p);
      break;
    }
    case 128:
      return KIND == kG1 ? launch_gemm1_tile(p, s) : launch_gemm2_tile(p, s);
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
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
  const size_t total = (size_t)p.T * (kHidden / 4);
  size_t grid = (total + 255) / 256;
  const size_t cap = (size_t)num_cus() * 8;
  if (grid > cap) grid = cap;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace moe
