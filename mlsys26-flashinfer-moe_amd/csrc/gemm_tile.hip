// Large-batch grouped fp8 block-scale GEMMs of the MoE layer (gfx950 MFMA).
//
// Tile = (work item of <= 128 assignment rows of one local expert) x (256 weight rows).
// A work-group of 8 wavefronts (two per SIMD) computes one tile; wavefront w = 4a + b owns
// weight rows [64b, 64b+64) of the tile (four 16-row MFMA fragments) against item rows
// [64a, 64a+64) (up to four 16-row groups): 4 x NG v_mfma_f32_16x16x128_f8f6f4 per 128-wide
// K-step with 16*NG fp32 accumulators per lane.
//   GEMM1: the tile is 128 SwiGLU columns: tile rows 0..127 are their gate rows of W13,
//          rows 128..255 the matching up rows; wavefront (a, b) owns columns [32b, 32b+32)
//          (fragments 0,1 gate, 2,3 up).
//   GEMM2: the tile is 256 hidden rows of W2.
// Both operands of a K-step (256 x 128 weight bytes, 128 x 128 activation bytes and the
// activations' scales) flow through a 3-stage LDS ring filled with global_load_lds two
// K-steps ahead: every 16-byte DMA instruction reads 8 whole 128-byte rows, so the vector
// memory pipeline sees full cache lines. The waits are explicit: at the top of step k every
// wave waits until only its loads of step k+1 are in flight (s_waitcnt vmcnt), then a raw
// s_barrier publishes stage k. Each K-step is one 128x128 scale block:
// acc += mfma * (s_a * s_w) (kernel.py:123-124, :234). With two wavefronts per SIMD, one
// wavefront's LDS reads and waits overlap the other's MFMAs. The four scale FMAs of an MFMA
// result are issued a row group (four MFMAs) after it, while later MFMAs run: VALU work that
// waits on the MFMA just issued leaves the matrix core idle (a loop that scales each result
// one MFMA later reaches ~62% of peak, four MFMAs later ~71%, against ~76% with no scaling).
//
// LDS tiles: 16-byte chunk c of row m lives at m*128 + ((c ^ ((m >> 1) & 7)) * 16), which
// spreads the 16 rows read by one ds_read_b128 across distinct bank groups.
//
// Scheduling: the work units (item, tile) of expert e are numbered tile-major
// (all items of one weight tile are consecutive) and dealt to the 8 XCDs in contiguous
// blocks, so the items sharing a weight tile run together on one XCD and reuse it from L2.
#include "moe_internal.h"
#include "moe_device.h"

namespace moe {

namespace {

constexpr int kTileRows = 128;                       // item rows per tile (max rows of an item)
constexpr int kTileW = 256;                          // weight rows per tile
constexpr int kTileWaves = 8;                        // wavefronts per work-group
constexpr int kStages = 3;                           // LDS ring stages
constexpr int kWDma = kTileW / kTileWaves / 8;       // weight DMA loads per wavefront per step (4)
constexpr int kADma = kTileRows / kTileWaves / 8;    // activation DMA loads per wavefront per step (2)
constexpr int kLoadsPerStep = kWDma + kADma + 1;     // + 1 scale DMA

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

struct TileStage {
  uint8_t w[kTileW * 128];
  uint8_t a[kTileRows * 128];
  float sa[kTileWaves * 64];   // scale of item row m at (m / 16) * 64 + m % 16
};

struct TileShared {
  TileStage st[kStages];
  float amax[4][kTileRows];
};

// Per-work-unit pointers of one lane.
struct TileCtx {
  const uint8_t* wbase;        // weight tensor (the per-step source is wbase + k*128 + woff)
  uint32_t woff[kWDma];        // weight DMA byte offsets (row + permuted 16-byte chunk); < 2^30
  const uint8_t* asrc[kADma];  // activation DMA sources
  const float* ssrc;           // activation scale DMA source
  size_t sstride;              // scale stride between K blocks
  const float* swp0;           // block scales of fragments 0,1 (GEMM1 gate) ...
  const float* swp1;           // ... and 2,3 (GEMM1 up)
  int r0, rows, tile;
};

// A 16-row MFMA operand fragment (rows m0 .. m0+15 of an LDS tile): lane l holds row
// m0 + l%16, chunks l/16 and 4 + l/16.
__device__ __forceinline__ v8i lds_frag(const uint8_t* buf, int m, int lane) {
  return join(*reinterpret_cast<const v4i*>(buf + swz(m, lane >> 4)),
              *reinterpret_cast<const v4i*>(buf + swz(m, 4 + (lane >> 4))));
}

template <bool G1, int NG>
__device__ __forceinline__ void tile_body(const GemmParams& p, const TileCtx& c, TileShared& sh) {
  constexpr int KS = G1 ? kHBlocks : kIBlocks;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wb = wave & 3, wa = wave >> 2;   // weight rows 64*wb.., item rows 64*wa..

  // lane k holds the weight block scales of K-step k (read back with readlane: the loop
  // itself touches no memory for them)
  const float sw0_lane = c.swp0[lane < KS ? lane : 0];
  const float sw1_lane = c.swp1[lane < KS ? lane : 0];

  // Loads of step k into stage s: this wave's share of the weight rows, activation rows and
  // activation scales. Every lane loads (lanes past the wave's 16 scale rows repeat them
  // into unused slots), so no load is divergent; every wave loads even if it has no rows.
  auto issue = [&](int k, int s) {
    TileStage& st = sh.st[s];
#pragma unroll
    for (int j = 0; j < kWDma; ++j) dma16(c.wbase + k * 128 + c.woff[j], &st.w[(32 * wave + 8 * j) * 128]);
#pragma unroll
    for (int j = 0; j < kADma; ++j) dma16(c.asrc[j] + k * 128, &st.a[(16 * wave + 8 * j) * 128]);
    dma4(c.ssrc + k * c.sstride, &st.sa[64 * wave]);
  };

  v4f acc[4][NG > 0 ? NG : 1];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[f][g] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};

  // weight fragment f of this wave: GEMM1 gate rows 32*wb + 16f (f = 0,1) and the up rows
  // 128 + 32*wb + 16(f-2) (f = 2,3); GEMM2 rows 64*wb + 16f
  auto wrow = [&](int f) {
    if constexpr (G1) return (f < 2 ? 32 * wb + 16 * f : 128 + 32 * wb + 16 * (f - 2)) + (lane & 15);
    else return 64 * wb + 16 * f + (lane & 15);
  };

  // The fragments a step starts with: its first row group and the four weight fragments.
  // They are read from LDS right after the barrier, before the step's DMA issue, so that
  // the issue overlaps their latency.
  struct Head {
    v8i wf[4];
    v8i bf;
    float sa;
  };
  auto load_head = [&](int s, Head& h) {
    if constexpr (NG > 0) {
      const TileStage& st = sh.st[s];
      h.bf = lds_frag(st.a, 64 * wa + (lane & 15), lane);
      h.sa = st.sa[(4 * wa) * 64 + (lane & 15)];
#pragma unroll
      for (int f = 0; f < 4; ++f) h.wf[f] = lds_frag(st.w, wrow(f), lane);
    }
  };

  // Software pipeline of the scale promotion: the MFMA results of a row group are scaled
  // and accumulated while the MFMAs of the next group run (the last group of a K-step while
  // the first group of the next step runs), so that the matrix core is not idle during the
  // VALU work. dp holds the pending group's MFMA results, p0/p1 its two scale products.
  v4f dp[4] = {zero, zero, zero, zero};
  float p0 = 0.f, p1 = 0.f;

  auto compute = [&](int s, const Head& h, float s0, float s1) __attribute__((always_inline)) {
    if constexpr (NG > 0) {
      const TileStage& st = sh.st[s];
      const v8i (&wf)[4] = h.wf;
      v8i bf = h.bf;
      float sa = h.sa;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        // the next row group's fragment is read from LDS while this group's MFMAs run
        v8i bf_next = bf;
        float sa_next = sa;
        if (g + 1 < NG) {
          bf_next = lds_frag(st.a, 64 * wa + 16 * (g + 1) + (lane & 15), lane);
          sa_next = st.sa[(4 * wa + g + 1) * 64 + (lane & 15)];
        }
        // pending group: the previous group of this step, or the previous step's last
        // group (zero results and zero scales before the first step)
        const int gp = g == 0 ? NG - 1 : g - 1;
        v4f d[4];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          d[f] = mfma16x16x128_fp8(wf[f], bf, zero);
          acc[f][gp] += dp[f] * (f < 2 ? p0 : p1);
        }
#pragma unroll
        for (int f = 0; f < 4; ++f) dp[f] = d[f];
        p0 = sa * s0;
        p1 = sa * s1;
        // two row groups' MFMA results live at a time (the scheduler would otherwise hoist
        // every MFMA of the step and hold all their results)
        __builtin_amdgcn_sched_barrier(0);
        bf = bf_next;
        sa = sa_next;
      }
    }
  };

  // the previous unit's readers of the LDS ring are done before it is refilled
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  issue(0, 0);
  issue(1, 1);
  int s_cur = 0, s_next = 2;
#pragma nounroll
  for (int k = 0; k < KS; ++k) {
    // step k's loads are complete for this wave (only step k+1's may be in flight), and
    // after the barrier for every wave; every wave is also done with stage s_next (step k-1)
    ring_barrier<kLoadsPerStep>();
    Head h;
    load_head(s_cur, h);
    __builtin_amdgcn_sched_barrier(0);
    issue(min(k + 2, KS - 1), s_next);   // past the last step: the last step again, never read
    __builtin_amdgcn_sched_barrier(0);
    const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw0_lane), k));
    const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw1_lane), k));
    compute(s_cur, h, s0, s1);
    s_cur = s_cur == kStages - 1 ? 0 : s_cur + 1;
    s_next = s_next == kStages - 1 ? 0 : s_next + 1;
  }
  // the last step's last row group
  if constexpr (NG > 0) {
#pragma unroll
    for (int f = 0; f < 4; ++f) acc[f][NG - 1] += dp[f] * (f < 2 ? p0 : p1);
  }
  // no ring load of this unit may land after the next unit starts refilling the ring
  wait_vmcnt<0>();

  if constexpr (G1) {
    // SwiGLU (kernel.py:126-129) and 1x128 requantisation (kernel.py:131-135 with 128
    // columns): the tile's 128 columns are one scale block, spread over the 4 wavefronts
    // that share this wave's item rows.
    float cval[NG > 0 ? NG : 1][2][4];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float amax = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x1 = acc[h][g][i], x2 = acc[2 + h][g][i];
          cval[g][h][i] = (x2 / (1.0f + __expf(-x2))) * x1;
          amax = fmaxf(amax, fabsf(cval[g][h][i]));
        }
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      if (lane < 16) sh.amax[wb][64 * wa + 16 * g + lane] = amax;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int m = 64 * wa + 16 * g + (lane & 15);
      const float amax = fmaxf(fmaxf(sh.amax[0][m], sh.amax[1][m]), fmaxf(sh.amax[2][m], sh.amax[3][m]));
      const float scale = fmaxf(amax / 448.0f, 1e-12f);
      if (m < c.rows) {
        uint8_t* dst = p.act + (size_t)(c.r0 + m) * kInter + c.tile * 128 + 32 * wb + 4 * (lane >> 4);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<uint32_t*>(dst + 16 * h) =
              pack_fp8x4(cval[g][h][0] / scale, cval[g][h][1] / scale, cval[g][h][2] / scale, cval[g][h][3] / scale);
        if (wb == 0 && lane < 16) p.act_scale[(size_t)(c.r0 + m) * kIBlocks + c.tile] = scale;
      }
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int m = 64 * wa + 16 * g + (lane & 15);
      if (m < c.rows) {
        const int pr = c.r0 + m;
        const int t = p.sorted_token[pr];
        const float wt = p.sorted_weight[pr];
        const bool direct = p.token_nlocal[t] == 1;
        const size_t slot = (size_t)p.sorted_slot[pr];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          const v4f val = acc[f][g] * wt;
          const int h = c.tile * kTileW + 64 * wb + 16 * f + 4 * (lane >> 4);
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

template <bool G1>
__global__ __launch_bounds__(kTileWaves * 64, 1) void gemm_tile_kernel(GemmParams p) {
  constexpr int TILES = (G1 ? 2 * kInter : kHidden) / kTileW;
  __shared__ __attribute__((aligned(1024))) TileShared sh;

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
    TileCtx c;
    c.r0 = __builtin_amdgcn_readfirstlane(it.y);
    c.rows = __builtin_amdgcn_readfirstlane(it.z);
    c.tile = __builtin_amdgcn_readfirstlane(v / ne);

    c.wbase = G1 ? p.w13 : p.w2;
    // DMA j of this wave fills 8 tile rows, lane l writing row +l/8, physical chunk l%8
    // (activation rows past the item's end repeat its first row)
#pragma unroll
    for (int j = 0; j < kWDma; ++j) {
      const int r = 32 * wave + 8 * j + (lane >> 3);
      const int ch = (lane & 7) ^ ((r >> 1) & 7);
      size_t grow;
      if constexpr (G1) grow = (size_t)e * 2 * kInter + (r < 128 ? c.tile * 128 + r : kInter + c.tile * 128 + r - 128);
      else grow = (size_t)e * kHidden + c.tile * kTileW + r;
      c.woff[j] = (uint32_t)(grow * (G1 ? kHidden : kInter) + ch * 16);
    }
#pragma unroll
    for (int j = 0; j < kADma; ++j) {
      const int m = 16 * wave + 8 * j + (lane >> 3);
      const int mm = m < c.rows ? m : 0;
      const int ch = (lane & 7) ^ ((m >> 1) & 7);
      size_t row;
      if constexpr (G1) row = (size_t)p.sorted_token[c.r0 + mm] * kHidden;
      else row = (size_t)(c.r0 + mm) * kInter;
      c.asrc[j] = (G1 ? p.hidden : p.act) + row + ch * 16;
    }
    {
      const int m = 16 * wave + (lane & 15);
      const int mm = m < c.rows ? m : 0;
      if constexpr (G1) c.ssrc = p.hidden_scale + p.sorted_token[c.r0 + mm];
      else c.ssrc = p.act_scale + (size_t)(c.r0 + mm) * kIBlocks;
      c.sstride = G1 ? (size_t)p.T : 1;
    }
    if constexpr (G1) {
      c.swp0 = p.w13_scale + ((size_t)e * 32 + c.tile) * kHBlocks;
      c.swp1 = p.w13_scale + ((size_t)e * 32 + kIBlocks + c.tile) * kHBlocks;
    } else {
      c.swp0 = p.w2_scale + ((size_t)e * kHBlocks + (c.tile * kTileW + 64 * (wave & 3)) / 128) * kIBlocks;
      c.swp1 = c.swp0;
    }
    // row groups of this wave's 64 item rows
    const int mine = c.rows - 64 * (wave >> 2);
    const int ng = mine <= 0 ? 0 : min(4, (mine + 15) >> 4);
    switch (ng) {
      case 0: tile_body<G1, 0>(p, c, sh); break;
      case 1: tile_body<G1, 1>(p, c, sh); break;
      case 2: tile_body<G1, 2>(p, c, sh); break;
      case 3: tile_body<G1, 3>(p, c, sh); break;
      default: tile_body<G1, 4>(p, c, sh); break;
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
  const int tiles = (G1 ? 2 * kInter : kHidden) / kTileW;
  const int max_units = p.max_items * tiles;
  int grid = (num_cus_tile() + 7) & ~7;
  const int cap = ((max_units + 7) / 8) * 8;
  if (grid > cap) grid = cap;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_tile_kernel<G1>), dim3(grid), dim3(kTileWaves * 64), 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm1_tile(const GemmParams& p, hipStream_t s) { return launch_tile<true>(p, s); }
hipError_t launch_gemm2_tile(const GemmParams& p, hipStream_t s) { return launch_tile<false>(p, s); }

}  // namespace moe
