// Large-batch grouped fp8 block-scale GEMMs of the MoE layer (gfx950 MFMA).
//
// Tile = (work item of <= 128 assignment rows of one local expert) x (WAVES*64 weight rows).
// Each wavefront of the work-group owns 64 weight rows (four 16-row MFMA fragments) against
// all rows of the item, i.e. 4 x NG v_mfma_f32_16x16x128_f8f6f4 per 128-wide K-step with
// 16*NG fp32 accumulators per lane (NG = row groups of 16 in the item; the K loop is
// instantiated per NG so that it carries no per-group branches).
//   GEMM1: wavefront w owns SwiGLU columns [32w, 32w+32) of the tile: gate rows and the
//          matching up rows (fragments 0,1 and 2,3).
//   GEMM2: wavefront w owns hidden rows [64w, 64w+64) of the tile.
// Activations (gathered by token for GEMM1, contiguous for GEMM2) and their per-K-block
// scales flow through a 3-stage LDS ring filled with global_load_lds (no VGPR staging),
// two K-steps ahead; weights stream straight into a 2-stage VGPR ring, one K-step ahead.
// The waits are explicit: at the top of step k every wave waits until only the ring
// loads of step k+1 are in flight (s_waitcnt vmcnt), then a raw s_barrier publishes the
// LDS stage of step k. Each K-step is one 128x128 scale block: acc += mfma * (s_a * s_w)
// (kernel.py:123-124, :234).
//
// LDS activation tile: 16-byte chunk c of row m lives at m*128 + ((c ^ ((m >> 1) & 7)) * 16),
// which spreads the 16 rows read by one ds_read_b128 across distinct bank groups.
//
// Scheduling: the work units (item, tile) of expert e are numbered tile-major
// (all items of one weight tile are consecutive) and dealt to the 8 XCDs in contiguous
// blocks, so the items sharing a weight tile run together on one XCD and reuse it from L2.
#include "moe_internal.h"
#include "moe_device.h"

namespace moe {

namespace {

constexpr int kTileRows = 128;   // LDS activation tile rows (max rows of a work item)
constexpr int kTileWaves = 4;    // wavefronts per work-group (one per SIMD)

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz(int m, int c) { return m * 128 + ((c ^ ((m >> 1) & 7)) << 4); }

__device__ __forceinline__ void dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_dst, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_dst, 4, 0, 0);
}

// vmcnt(n) with expcnt and lgkmcnt left unconstrained (gfx9 s_waitcnt encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(N | (7 << 4) | (15 << 8));
}

// Work-group barrier that publishes LDS ring stages filled by global_load_lds: the caller's
// vmcnt wait covers this wave's loads, s_barrier covers the other waves', and the two
// compiler-only fences keep every memory access on its side of the barrier.
template <int N>
__device__ __forceinline__ void ring_barrier() {
  wait_vmcnt<N>();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ v8i load_frag(const uint8_t* p) {
  const v4i lo = *reinterpret_cast<const v4i*>(p);
  const v4i hi = *reinterpret_cast<const v4i*>(p + 64);
  return join(lo, hi);
}

constexpr int kStages = 4;       // LDS ring stages (4 divides both K-step counts, 56 and 16)

template <int WAVES>
struct TileShared {
  uint8_t a[kStages][kTileRows * 128];
  float sa[kStages][WAVES * 64];   // row m at (m / DMA_ROWS) * 64 + m % DMA_ROWS
  float amax[WAVES][kTileRows];
};

template <int V>
struct IntC {
  static constexpr int value = V;
};

// Per-work-unit pointers of one lane.
template <int NDMA>
struct TileCtx {
  const uint8_t* asrc[NDMA];  // activation DMA sources (row + permuted 16-byte chunk)
  const float* ssrc;          // activation scale DMA source
  size_t sstride;             // scale stride between K blocks
  const uint8_t* wp[4];       // weight fragment rows
  const float* swp0;          // block scales of fragments 0,1 (GEMM1 gate) ...
  const float* swp1;          // ... and 2,3 (GEMM1 up)
  int r0, rows, tile;
};

template <bool G1, int WAVES, int NG>
__device__ __forceinline__ void tile_body(const GemmParams& p, const TileCtx<kTileRows / WAVES / 8>& c,
                                          TileShared<WAVES>& sh) {
  constexpr int KS = G1 ? kHBlocks : kIBlocks;
  constexpr int TILE_W = WAVES * 64;
  constexpr int DMA_ROWS = kTileRows / WAVES;
  constexpr int NDMA = DMA_ROWS / 8;
  constexpr int DMA_PER_STEP = NDMA + 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // every lane of the wave loads (lanes >= DMA_ROWS repeat a row into unused slots), so
  // the loads carry no divergent control flow
  auto issue_a = [&](int k, int stage) {
#pragma unroll
    for (int j = 0; j < NDMA; ++j)
      dma16(c.asrc[j] + k * 128, &sh.a[stage][(DMA_ROWS * wave + 8 * j) * 128]);
    dma4(c.ssrc + k * c.sstride, &sh.sa[stage][64 * wave]);
  };
  // lane k holds the weight block scales of K-step k (read back with readlane: the loop
  // itself touches no memory for them)
  const float sw0_lane = c.swp0[lane < KS ? lane : 0];
  const float sw1_lane = c.swp1[lane < KS ? lane : 0];
  v8i wr[2][4];
  auto load_w = [&](int k, v8i (&dst)[4]) {
#pragma unroll
    for (int f = 0; f < 4; ++f) dst[f] = load_frag(c.wp[f] + k * 128);
  };
  v4f acc[4][NG];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[f][g] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int stage, const v8i (&wf)[4], float s0, float s1) {
    const uint8_t* abuf = sh.a[stage];
    const float* sbuf = sh.sa[stage];
    const int c0 = lane >> 4, c1 = 4 + (lane >> 4);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int m = g * 16 + (lane & 15);
      const v8i bf = join(*reinterpret_cast<const v4i*>(abuf + swz(m, c0)),
                          *reinterpret_cast<const v4i*>(abuf + swz(m, c1)));
      const float sa = sbuf[(m / DMA_ROWS) * 64 + m % DMA_ROWS];
      const float f0 = sa * s0, f1 = sa * s1;
      v4f d[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) d[f] = mfma16x16x128_fp8(wf[f], bf, zero);
#pragma unroll
      for (int f = 0; f < 4; ++f) acc[f][g] += d[f] * (f < 2 ? f0 : f1);
      // one row group's MFMA results live at a time (the scheduler would otherwise hoist
      // every MFMA of the step and hold all their results)
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One K-step. Issue order per step: weights of step k+1, then activations of step
  // k+3, so that at the top of step k only step k+2's activation loads may be in flight.
  // Every step has the same shape: past the last step, the loads repeat the last step's
  // data (cache-hot) into ring slots that are never read.
  auto step = [&](int k, auto UU) {
    constexpr int uu = decltype(UU)::value;   // k % 4
    ring_barrier<DMA_PER_STEP>();
    load_w(min(k + 1, KS - 1), wr[(uu + 1) & 1]);
    issue_a(min(k + 3, KS - 1), (uu + 3) % kStages);
    const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw0_lane), k));
    const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw1_lane), k));
    compute(uu, wr[uu & 1], s0, s1);
  };

  // the previous unit's readers of the LDS ring are done before it is refilled
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  issue_a(0, 0);
  issue_a(1, 1);
  issue_a(2, 2);
  load_w(0, wr[0]);
  // the vmcnt wait at step 0 (DMA_PER_STEP outstanding) then also covers stages 0 and 1
  static_assert(KS % kStages == 0, "K-step count");
#pragma nounroll
  for (int k0 = 0; k0 < KS; k0 += kStages) {
    step(k0 + 0, IntC<0>{});
    step(k0 + 1, IntC<1>{});
    step(k0 + 2, IntC<2>{});
    step(k0 + 3, IntC<3>{});
  }
  // no ring load of this unit may land after the next unit starts refilling the ring
  wait_vmcnt<0>();

  if constexpr (G1) {
    // SwiGLU (kernel.py:126-129) and 1x128 requantisation (kernel.py:131-135 with 128 columns).
    // Pass 1 publishes each row's amax over this wave's 32 columns; pass 2 recomputes the
    // SwiGLU values (cheaper than keeping them live) and quantises with the block scale.
    auto swiglu = [&](int h, int g, int i) {
      const float x1 = acc[h][g][i], x2 = acc[2 + h][g][i];
      return (x2 / (1.0f + __expf(-x2))) * x1;
    };
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float amax = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(swiglu(h, g, i)));
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      if (lane < 16) sh.amax[wave][g * 16 + lane] = amax;
    }
    __syncthreads();
    const int wb = wave & ~3;   // the 4 wavefronts sharing a 128-column scale block
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int m = g * 16 + (lane & 15);
      const float amax = fmaxf(fmaxf(sh.amax[wb][m], sh.amax[wb + 1][m]), fmaxf(sh.amax[wb + 2][m], sh.amax[wb + 3][m]));
      const float scale = fmaxf(amax / 448.0f, 1e-12f);
      if (m < c.rows) {
        const int col = c.tile * (TILE_W / 2) + wave * 32;
        uint8_t* dst = p.act + (size_t)(c.r0 + m) * kInter + col + 4 * (lane >> 4);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<uint32_t*>(dst + 16 * h) =
              pack_fp8x4(swiglu(h, g, 0) / scale, swiglu(h, g, 1) / scale, swiglu(h, g, 2) / scale,
                         swiglu(h, g, 3) / scale);
        if ((wave & 3) == 0 && lane < 16) p.act_scale[(size_t)(c.r0 + m) * kIBlocks + col / 128] = scale;
      }
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int m = g * 16 + (lane & 15);
      if (m < c.rows) {
        const int pr = c.r0 + m;
        const int t = p.sorted_token[pr];
        const float wt = p.sorted_weight[pr];
        const bool direct = p.token_nlocal[t] == 1;
        const size_t slot = (size_t)p.sorted_slot[pr];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          const v4f val = acc[f][g] * wt;
          const int h = c.tile * TILE_W + wave * 64 + f * 16 + 4 * (lane >> 4);
          if (direct) {
            if (p.out_dtype == MOE_FP8_OUT_BF16)
              *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + (size_t)t * kHidden + h) =
                  pack_bf16x4(val[0], val[1], val[2], val[3]);
            else
              *reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.out) + (size_t)t * kHidden + h) = val;
          } else {
            *reinterpret_cast<v4f*>(p.partial + slot * kHidden + h) = val;
          }
        }
      }
    }
  }
}

template <bool G1, int WAVES>
__global__ __launch_bounds__(WAVES * 64, 1) void gemm_tile_kernel(GemmParams p) {
  constexpr int TILE_W = WAVES * 64;
  constexpr int TILES = (G1 ? 2 * kInter : kHidden) / TILE_W;
  constexpr int DMA_ROWS = kTileRows / WAVES;
  constexpr int NDMA = DMA_ROWS / 8;
  static_assert(DMA_ROWS <= 64 && NDMA >= 1, "activation loader shape");
  __shared__ __attribute__((aligned(1024))) TileShared<WAVES> sh;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n_items = min(p.counters[kCtrItems], p.max_items);
  const int units = n_items * TILES;
  const int per_xcd = (units + 7) >> 3;

  for (int w = blockIdx.x; w < 8 * per_xcd; w += gridDim.x) {
    const int u = (w & 7) * per_xcd + (w >> 3);
    if (u >= units) continue;
    const int q = u / TILES;
    const int qw = reinterpret_cast<const int4*>(p.work_items)[q].w;
    const int first = qw & 0xFFFF, ne = qw >> 16;
    const int v = u - first * TILES;
    const int4 it = reinterpret_cast<const int4*>(p.work_items)[first + v % ne];
    // work-item fields are wave-uniform; say so, so that everything derived from them
    // (notably the weight block-scale addresses) stays in scalar registers
    const int e = __builtin_amdgcn_readfirstlane(it.x);
    TileCtx<NDMA> c;
    c.r0 = __builtin_amdgcn_readfirstlane(it.y);
    c.rows = __builtin_amdgcn_readfirstlane(it.z);
    c.tile = __builtin_amdgcn_readfirstlane(v / ne);

    // activation DMA: load j of this wave fills LDS rows DMA_ROWS*w + 8j .. +8, lane l
    // writing row +l/8, physical chunk l%8 (rows past the item's end repeat its first row)
#pragma unroll
    for (int j = 0; j < NDMA; ++j) {
      const int m = DMA_ROWS * wave + 8 * j + (lane >> 3);
      const int mm = m < c.rows ? m : 0;
      const int ch = (lane & 7) ^ ((m >> 1) & 7);
      size_t row;
      if constexpr (G1) row = (size_t)p.sorted_token[c.r0 + mm] * kHidden;
      else row = (size_t)(c.r0 + mm) * kInter;
      c.asrc[j] = (G1 ? p.hidden : p.act) + row + ch * 16;
    }
    {
      const int m = DMA_ROWS * wave + (lane % DMA_ROWS);
      const int mm = m < c.rows ? m : 0;
      if constexpr (G1) c.ssrc = p.hidden_scale + p.sorted_token[c.r0 + mm];
      else c.ssrc = p.act_scale + (size_t)(c.r0 + mm) * kIBlocks;
      c.sstride = G1 ? (size_t)p.T : 1;
    }
    if constexpr (G1) {
      const int row = c.tile * (TILE_W / 2) + wave * 32 + (lane & 15);   // gate row; up = +I
      const uint8_t* base = p.w13 + ((size_t)e * 2 * kInter + row) * kHidden + (lane >> 4) * 16;
      c.wp[0] = base;
      c.wp[1] = base + (size_t)16 * kHidden;
      c.wp[2] = base + (size_t)kInter * kHidden;
      c.wp[3] = base + (size_t)(kInter + 16) * kHidden;
      const int blk = (c.tile * (TILE_W / 2) + wave * 32) / 128;
      c.swp0 = p.w13_scale + ((size_t)e * 32 + blk) * kHBlocks;
      c.swp1 = p.w13_scale + ((size_t)e * 32 + kIBlocks + blk) * kHBlocks;
    } else {
      const int row = c.tile * TILE_W + wave * 64 + (lane & 15);
      const uint8_t* base = p.w2 + ((size_t)e * kHidden + row) * kInter + (lane >> 4) * 16;
#pragma unroll
      for (int f = 0; f < 4; ++f) c.wp[f] = base + (size_t)(16 * f) * kInter;
      c.swp0 = p.w2_scale + ((size_t)e * kHBlocks + (c.tile * TILE_W + wave * 64) / 128) * kIBlocks;
      c.swp1 = c.swp0;
    }
    switch ((c.rows + 15) >> 4) {
      case 1: tile_body<G1, WAVES, 1>(p, c, sh); break;
      case 2: tile_body<G1, WAVES, 2>(p, c, sh); break;
      case 3: tile_body<G1, WAVES, 3>(p, c, sh); break;
      case 4: tile_body<G1, WAVES, 4>(p, c, sh); break;
      case 5: tile_body<G1, WAVES, 5>(p, c, sh); break;
      case 6: tile_body<G1, WAVES, 6>(p, c, sh); break;
      case 7: tile_body<G1, WAVES, 7>(p, c, sh); break;
      default: tile_body<G1, WAVES, 8>(p, c, sh); break;
    }
  }
}

int num_cus_tile() {
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

template <bool G1>
hipError_t launch_tile(const GemmParams& p, hipStream_t s) {
  const int tiles = (G1 ? 2 * kInter : kHidden) / (kTileWaves * 64);
  const int max_units = p.max_items * tiles;
  int grid = (num_cus_tile() + 7) & ~7;
  const int cap = ((max_units + 7) / 8) * 8;
  if (grid > cap) grid = cap;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_tile_kernel<G1, kTileWaves>), dim3(grid), dim3(kTileWaves * 64), 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm1_tile(const GemmParams& p, hipStream_t s) { return launch_tile<true>(p, s); }
hipError_t launch_gemm2_tile(const GemmParams& p, hipStream_t s) { return launch_tile<false>(p, s); }

}  // namespace moe
