// Large-batch grouped fp8 block-scale GEMMs of the MoE layer (gfx950 MFMA).
//
// Tile = (work item of one local expert) x (256 weight rows). Two instances: items of up to
// 128 rows (T < 4096) and of up to 160 rows (T >= 4096; the largest whose three ring stages
// fit the CU's LDS). The bigger the item, the fewer bytes the CU moves per flop, which is
// what bounds this loop at large T; at mid-size T the fewer, longer units of the large
// instance would balance worse over the CUs.
// A work-group of 8 wavefronts (two per SIMD) computes one tile; wavefront w = 4a + b owns
// weight rows [64b, 64b+64) of the tile (four 16-row MFMA fragments) against half a of the
// item's 16-row groups (up to five; the halves differ by at most one group):
// 4 x NG v_mfma_f32_16x16x128_f8f6f4 per 128-wide K-step with 16*NG fp32 accumulators per
// lane.
//   GEMM1: the tile is 128 SwiGLU columns: tile rows 0..127 are their gate rows of W13,
//          rows 128..255 the matching up rows; wavefront (a, b) owns columns [32b, 32b+32)
//          (fragments 0,1 gate, 2,3 up).
//   GEMM2: the tile is 256 hidden rows of W2.
// Both operands of a K-step (256 x 128 weight bytes, 128 or 160 x 128 activation bytes and
// the activations' scales) flow through a 3-stage LDS ring (146 or 158 KB) filled with
// global_load_lds two K-steps ahead: every 16-byte DMA instruction reads 8 whole 128-byte
// rows, so the vector memory pipeline sees full cache lines. The waits are explicit: at the
// top of step k every wave waits until only its loads of step k+1 are in flight (s_waitcnt
// vmcnt), then a raw s_barrier publishes stage k. Every wave issues the same number of loads
// each step and the loop has no data-dependent branch (the last two steps reload the last
// step into stages nobody reads): a loop split into blocks by per-wave load counts measured
// 15% slower at T=1024. Each K-step is one 128x128 scale block:
// acc += mfma * (s_a * s_w) (kernel.py:123-124, :234). With two wavefronts per SIMD, one
// wavefront's LDS reads and waits overlap the other's MFMAs. The four scale FMAs of an MFMA
// result are issued a row group (four MFMAs) after it, while later MFMAs run: VALU work that
// waits on the MFMA just issued leaves the matrix core idle (a loop that scales each result
// one MFMA later reaches ~62% of peak, four MFMAs later ~71%, against ~76% with no scaling).
//
// LDS tiles: 16-byte chunk c of row m lives at m*128 + ((c ^ ((m >> 1) & 7)) * 16), which
// spreads the 16 rows read by one ds_read_b128 across distinct bank groups.
//
// Scheduling: the work units (item, tile) of expert e are numbered tile-major (all items of
// one weight tile are consecutive); the items sharing a weight tile run together on one XCD
// and reuse it from L2 (the work runs follow this numbering, the per-XCD lists take an
// expert's units on their XCD item by item). A work-group claims its next unit on a 64-bit
// per-XCD counter while its current unit runs; the experts' item geometry is read once per
// launch into lane registers, so a unit's setup makes no dependent memory round trip.
//   Per-XCD lists (GEMM1; GEMM2 with items of up to 128 rows): XCD x takes weight tiles
//          t0, t0 + 8, .. of every expert, t0 = (x - 4 * (rank % 2)) % 8 for the expert's rank
//          by descending item rows, so that every XCD gets the same mix of long and short
//          units; its work-groups take the units of that list, longest experts first, from the
//          XCD's counter as they finish. Inside an expert the list goes item by item (the
//          item's 2 GEMM1 or 3-4 GEMM2 tiles of this XCD, then the next item's), so that the
//          units running together share their items' activation rows as well as their weight
//          tiles: on the skewed T=4096 batch (experts of 26 items) GEMM1 fetches 2.34 instead
//          of 3.13 GB per launch from outside the L2s (tile by tile, the rows of 26 items
//          outgrew the L2 before the XCD's second tile reread them), 656 against 664 us; no
//          change at T=8192 or T=1024. GEMM2 reserves one entry ahead, so that a unit
//          knows the next one in time to prefetch its first K-steps. Measured against
//          contiguous blocks of units per XCD: GEMM1 296 against 313 us at T=8192, 164
//          against 174 at T=1024, 656 against 682 on the skewed T=4096 batch; GEMM2 +
//          combine 114 against 123 us at T=1024.
//   Work runs with stealing (GEMM2 with items of up to 160 rows): XCD x owns a contiguous run
//          of the unit numbering, cut at weight-tile boundaries where the estimated work (item
//          rows plus a fixed cost per unit) reaches x/8 and (x+1)/8 of the launch's; its
//          work-groups claim the run's units in order from the front of the XCD's counter.
//          Once a run is used up its work-groups take units from the back of the run with the
//          most units left: the counter's high half counts those, and a claim is good while
//          the two halves together stay below the run's length, so every unit runs exactly
//          once. Against contiguous equal blocks of units fixed in advance: GEMM2 + combine
//          234.8 against 239.7 us at T=8192 (the XCDs end within 10 us of each other instead of
//          28), 542 against 537 us on the skewed batch, whose GEMM1 gains 3 us from the unit
//          setup without memory round trips. The cut estimate alone, without stealing, measured
//          +13 us on the skewed batch: the XCDs' unit times differ by 5% with the load on their
//          L2s, which no estimate made before the launch knows.
#include <atomic>

#include "moe_internal.h"
#include "moe_device.h"

namespace moe {

namespace {

constexpr int kTileW = 256;                          // weight rows per tile
constexpr int kTileWaves = 8;                        // wavefronts per work-group
constexpr int kStages = 3;                           // LDS ring stages
constexpr int kWDma = kTileW / kTileWaves / 8;       // weight DMA loads per wavefront per step (4)

// Shape of the kernel for items of up to ROWS rows (kTileItemRowsMid or kTileItemRowsLarge).
// Per K-step every wavefront issues kLoadsPerStep loads: its 32 weight rows (kWDma loads),
// the activation row blocks w and w+8 of the tile (8 rows each) and a third load:
//   128 rows: the scales of one 64-row block: GEMM1 block w%4, GEMM2 block (w/2)%4 and
//             64-column half w%2 of the K-step (both capped at the last block; a load that
//             repeats another writes the same bytes to the same LDS slots);
//   160 rows: activation block w+16 for waves 0-3, and the scales of 64-row block w-4
//             (capped at the last one) for waves 4-7.
// Columns per requantisation scale of GEMM1's output (kQCols): the reference's 64
// (kernel.py:131-135) with 128-row items, so that GEMM2 applies two activation scales per
// 128-wide K-step: it runs v_mfma_f32_32x32x64_f8f6f4 on 32-row item groups, one MFMA per
// 64-column half (against two 16x16x128 MFMAs per fragment with the other half's bytes
// zeroed: the same time at T=1024, half the matrix-core work); 128 with 160-row items
// (T >= 4096), one scale and one 16x16x128 MFMA per fragment. Measured with 64 there too:
// GEMM2 + combine at T=8192 238-242 -> 274-283 us and on the skewed T=4096 batch 539-542 ->
// 623-625 us with 32x32x64 MFMAs on 32-row groups (both halves' scales row-interleaved in LDS,
// an eighth load per wavefront and K-step, 256 registers), 249 -> 323 and 552 -> 732 with
// the zeroed-half 16x16x128 form: the doubled scale promotion costs what remains.
template <int ROWS>
struct TileShape {
  static constexpr int kRows = ROWS;
  static constexpr int kABlocks = ROWS / 8;
  static constexpr bool kThirdBlock = kABlocks > 2 * kTileWaves;   // waves 0-3 load block w+16
  static constexpr int kSBlocks = (ROWS + 63) / 64;       // 64-row scale blocks
  static constexpr int kSSlots = 64 * kSBlocks;
  static constexpr int kQCols = ROWS == kTileItemRowsMid ? 64 : 128;
  static constexpr int kQBlocks = kInter / kQCols;        // activation scales per row
  static constexpr int kSHalves = kBlock / kQCols;        // GEMM2 activation scales per K-step
  static constexpr int kMaxNG = (ROWS / 16 + 1) / 2;      // row groups of a wavefront half
  // GEMM2 with two activation scales per K-step: v_mfma_f32_32x32x64_f8f6f4, one MFMA per
  // 64-wide half of the K-step, on 32-row item groups (kW32)
  static constexpr bool kW32 = kSHalves == 2;
  static constexpr int kMaxNG32 = (ROWS / 32 + 1) / 2;    // 32-row groups of a wavefront half
  static constexpr int kLoadsPerStep = kWDma + 3;
  static_assert(ROWS % 16 == 0 && (kABlocks == 2 * kTileWaves || kABlocks == 2 * kTileWaves + 4), "tile rows");
  static_assert(kSBlocks <= 4, "scale blocks");
  static_assert(kSHalves == 1 || !kThirdBlock, "two scale halves only with the 128-row load plan");
};

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

// waits for this wave's LDS operations only (vmcnt 63, expcnt 7, lgkmcnt 0)
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14)); }

template <int ROWS>
struct TileStage {
  uint8_t w[kTileW * 128];
  uint8_t a[ROWS * 128];
  // scale of item row m at m (GEMM2 with two per K-step: the second half's at kSSlots + m)
  float sa[TileShape<ROWS>::kSHalves * TileShape<ROWS>::kSSlots];
};

// The ring and the next list entry share one LDS object: with a second __shared__
// variable the compiler no longer tells the ring's DMA writes from its reads and waits for
// every load in flight before each LDS read.
template <int ROWS>
struct TileShared {
  TileStage<ROWS> st[kStages];
  unsigned long long next;   // the claim counter's value before this work-group's last claim
  int stolen;                // a unit taken from another XCD's run, or -1
  int steal_from;            // that XCD
};
static_assert(sizeof(TileShared<kTileItemRowsLarge>) <= 160 * 1024 && sizeof(TileShared<kTileItemRowsMid>) <= 160 * 1024,
              "LDS of one CU");
static_assert(4 * kTileItemRowsLarge * sizeof(float) <= kTileW * 128, "amax fits in a weight tile");

// Per-work-unit pointers of one lane.
template <int ROWS>
struct TileCtx {
  const uint8_t* wbase;        // weight tensor (the per-step source is wbase + k*128 + woff)
  uint32_t woff[kWDma];        // weight DMA byte offsets (row + permuted 16-byte chunk); < 2^30
  const uint8_t* asrc[3];      // activation DMA sources of blocks w, w+8 (and w+16)
  int sblk;                    // the 64-row scale block this wave loads
  int shalf;                   // GEMM2 with 64-column scales: the half of the K-step it loads
  const float* ssrc;           // activation scale DMA source (waves 4-7)
  size_t sstride;              // scale stride between K blocks
  float sw0_lane, sw1_lane;     // lane k: weight block scale of K-step k of fragments 0,1
                               // (GEMM1 gate) and 2,3 (GEMM1 up)
  int r0, rows, tile, m0;      // item rows [r0, r0+rows); first item row of this wave's half
  int ng;                      // row groups of this wave's half
  // GEMM2: the destination (token, or -1 - flat slot) and routing weight of the lane's row in
  // each of this wave's row groups, loaded when the unit is set up (a unit ahead) so that the
  // epilogue makes no memory round trip for them (rows past the item read its first row)
  int dest[TileShape<ROWS>::kW32 ? TileShape<ROWS>::kMaxNG32 : TileShape<ROWS>::kMaxNG];
  float wt[TileShape<ROWS>::kW32 ? TileShape<ROWS>::kMaxNG32 : TileShape<ROWS>::kMaxNG];
};

// A 16-row MFMA operand fragment (rows m0 .. m0+15 of an LDS tile): lane l holds row
// m0 + l%16, chunks l/16 and 4 + l/16.
__device__ __forceinline__ v8i lds_frag(const uint8_t* buf, int m, int lane) {
  return join(*reinterpret_cast<const v4i*>(buf + swz(m, lane >> 4)),
              *reinterpret_cast<const v4i*>(buf + swz(m, 4 + (lane >> 4))));
}

// A 32-row operand of one 64-wide half hh of a K-step (rows m0 .. m0+31 of an LDS tile, for
// v_mfma_f32_32x32x64_f8f6f4): lane l holds row m0 + l%32, chunks 4hh + 2(l/32) and the next.
__device__ __forceinline__ v8i lds_frag32(const uint8_t* buf, int m, int hh, int lane) {
  const int c = 4 * hh + 2 * (lane >> 5);
  return join(*reinterpret_cast<const v4i*>(buf + swz(m, c)), *reinterpret_cast<const v4i*>(buf + swz(m, c + 1)));
}

// One unit (c). Its K-steps read ring stages s_base, s_base+1, .. (mod 3). GEMM2 (16 K-steps
// per unit) prefetches across units: its last two steps load the first two steps of the next
// unit (n) when `have_n`, and `pre` says that this unit's were loaded so. GEMM1 (56 K-steps)
// does not (the per-step address selects cost it more than the saved ring fill): its last two
// steps, like GEMM2's last unit's, load the last step again into stages nobody reads.
template <bool G1, int NG, int ROWS>
__device__ __forceinline__ void tile_body(const GemmParams& p, const TileCtx<ROWS>& c, const TileCtx<ROWS>& n,
                                          bool have_n, int s_base, bool pre, TileShared<ROWS>& sh,
                                          unsigned long long* claim, unsigned long long inc) {
  using S = TileShape<ROWS>;
  constexpr int KS = G1 ? kHBlocks : kIBlocks;
  // GEMM2 with two activation scales per K-step (64-column requantisation blocks): 32x32x64
  // MFMAs, NG counts 32-row item groups
  constexpr bool W32 = !G1 && S::kW32;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wb = wave & 3;     // weight rows 64*wb.. (item rows: the wave's half, from c.m0)

  // lane k holds the weight block scales of K-step k (read back with readlane: the loop
  // itself touches no memory for them)
  const float sw0_lane = c.sw0_lane;
  const float sw1_lane = c.sw1_lane;

  // Loads of unit step kk into stage s: this wave's share of the weight rows, activation
  // rows and activation scales, S::kLoadsPerStep in all. Steps past the unit's last are the
  // next unit's first ones (or, without a next unit, the last step again); the choice is a
  // select of the source addresses, so the loop has no branch. Every lane loads (activation
  // rows and scale rows past the item's end repeat its first row into slots nobody reads), so
  // no load is divergent; every wave loads even if it has no rows.
  auto issue = [&](int kk, int s) __attribute__((always_inline)) {
    const bool nxt = !G1 && kk >= KS && have_n;
    const int k = kk < KS ? kk : (nxt ? kk - KS : KS - 1);
    TileStage<ROWS>& st = sh.st[s];
    const uint8_t* wk = (nxt ? n.wbase : c.wbase) + k * 128;
#pragma unroll
    for (int j = 0; j < kWDma; ++j) dma16(wk + (nxt ? n.woff[j] : c.woff[j]), &st.w[(32 * wave + 8 * j) * 128]);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16((nxt ? n.asrc[j] : c.asrc[j]) + k * 128, &st.a[8 * (wave + kTileWaves * j) * 128]);
    const float* sk = (nxt ? n.ssrc : c.ssrc) + k * c.sstride;
    if constexpr (S::kThirdBlock) {
      if (wave < 4) dma16((nxt ? n.asrc[2] : c.asrc[2]) + k * 128, &st.a[8 * (wave + 2 * kTileWaves) * 128]);
      else dma4(sk, &st.sa[64 * c.sblk]);
    } else {
      dma4(sk, &st.sa[S::kSSlots * c.shalf + 64 * c.sblk]);
    }
  };

  constexpr int NG1 = NG > 0 ? NG : 1;
  v4f acc[W32 ? 1 : 4][W32 ? 1 : NG1];
  v16f acc32[W32 ? 2 : 1][W32 ? NG1 : 1];   // W32: [weight rows 32*blk..][item group]
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  const v16f zero16 = {};
  if constexpr (W32) {
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int g = 0; g < NG; ++g) acc32[blk][g] = zero16;
  } else {
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int g = 0; g < NG; ++g) acc[f][g] = zero;
  }

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
      const TileStage<ROWS>& st = sh.st[s];
      h.bf = lds_frag(st.a + c.m0 * 128, lane & 15, lane);
      h.sa = st.sa[c.m0 + (lane & 15)];
#pragma unroll
      for (int f = 0; f < 4; ++f) h.wf[f] = lds_frag(st.w, wrow(f), lane);
    }
  };
  // W32: the wave's two 32-row weight blocks and its first item group, each as two 64-wide
  // halves, and that group's two activation scales
  struct Head32 {
    v8i wf[2][2];
    v8i bf[2];
    float sa[2];
  };
  auto load_head32 = [&](int s, Head32& h) {
    if constexpr (NG > 0) {
      const TileStage<ROWS>& st = sh.st[s];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        h.bf[hh] = lds_frag32(st.a, c.m0 + (lane & 31), hh, lane);
        h.sa[hh] = st.sa[S::kSSlots * hh + c.m0 + (lane & 31)];
      }
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) h.wf[blk][hh] = lds_frag32(st.w, 64 * wb + 32 * blk + (lane & 31), hh, lane);
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
      const TileStage<ROWS>& st = sh.st[s];
      const v8i (&wf)[4] = h.wf;
      v8i bf = h.bf;
      float sa = h.sa;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        // the next row group's fragment is read from LDS while this group's MFMAs run
        v8i bf_next = bf;
        float sa_next = sa;
        if (g + 1 < NG) {
          bf_next = lds_frag(st.a + c.m0 * 128, 16 * (g + 1) + (lane & 15), lane);
          sa_next = st.sa[c.m0 + 16 * (g + 1) + (lane & 15)];
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

  // W32: per item group the four MFMAs (two weight blocks x two K halves) first, then their
  // scale promotion, acc += d_h * (s_act,h * s_w), in issue order, so that each FMA finds its
  // MFMA done; the next group's fragment and scales are read from LDS meanwhile.
  auto compute32 = [&](int s, const Head32& h, float s0) __attribute__((always_inline)) {
    if constexpr (NG > 0) {
      const TileStage<ROWS>& st = sh.st[s];
      v8i bf[2] = {h.bf[0], h.bf[1]};
      float sa[2] = {h.sa[0], h.sa[1]};
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        v8i bf_next[2] = {bf[0], bf[1]};
        float sa_next[2] = {sa[0], sa[1]};
        if (g + 1 < NG) {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            bf_next[hh] = lds_frag32(st.a, c.m0 + 32 * (g + 1) + (lane & 31), hh, lane);
            sa_next[hh] = st.sa[S::kSSlots * hh + c.m0 + 32 * (g + 1) + (lane & 31)];
          }
        }
        v16f d[2][2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) d[blk][hh] = mfma32x32x64_fp8(h.wf[blk][hh], bf[hh], zero16);
        const float q0 = sa[0] * s0, q1 = sa[1] * s0;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          acc32[blk][g] += d[blk][0] * q0;
          acc32[blk][g] += d[blk][1] * q1;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          bf[hh] = bf_next[hh];
          sa[hh] = sa_next[hh];
        }
      }
    }
  };

  // A unit whose first two steps were not prefetched loads them itself, once every wave is
  // done with the ring (the previous unit's last loads have landed: see the end of the unit).
  int s_cur = s_base, s_next = s_base == 0 ? kStages - 1 : s_base - 1;
  if (!pre) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    issue(0, s_cur);
    issue(1, s_cur == kStages - 1 ? 0 : s_cur + 1);
  }
#pragma nounroll
  for (int k = 0; k < KS; ++k) {
    // step k's loads are complete for this wave (only step k+1's may be in flight), and
    // after the barrier for every wave; every wave is also done with stage s_next (step k-1).
    // A prefetched unit's first two steps landed before the previous unit's epilogue stored
    // anything (below): those steps do not wait, so the stores drain under their MFMAs (the
    // counter is in order, a wait for a later load waits for them).
    if (!pre || k >= 2) wait_vmcnt<S::kLoadsPerStep>();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw0_lane), k));
    if constexpr (W32) {
      Head32 h;
      load_head32(s_cur, h);
      __builtin_amdgcn_sched_barrier(0);
      issue(k + 2, s_next);
      __builtin_amdgcn_sched_barrier(0);
      compute32(s_cur, h, s0);
    } else {
      Head h;
      load_head(s_cur, h);
      __builtin_amdgcn_sched_barrier(0);
      issue(k + 2, s_next);
      __builtin_amdgcn_sched_barrier(0);
      const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw1_lane), k));
      compute(s_cur, h, s0, s1);
    }
    s_cur = s_cur == kStages - 1 ? 0 : s_cur + 1;
    s_next = s_next == kStages - 1 ? 0 : s_next + 1;
  }
  // the last step's last row group
  if constexpr (NG > 0 && !W32) {
#pragma unroll
    for (int f = 0; f < 4; ++f) acc[f][NG - 1] += dp[f] * (f < 2 ? p0 : p1);
  }
  // The loads in flight now are the next unit's first two steps, or reloads nobody reads; the
  // reloads must land before the next unit refills the ring.
  if (G1 || !have_n) wait_vmcnt<0>();
  // the work-group's next claim on a per-XCD counter (front or back); the counter's round trip
  // overlaps the epilogue
  unsigned long long got = 0;
  if (claim != nullptr && threadIdx.x == 0) got = atomicAdd(claim, inc);

  if constexpr (G1) {
    // SwiGLU (kernel.py:126-129) and requantisation per S::kQCols columns (kernel.py:131-135):
    // the tile's 128 columns are spread over the 4 wavefronts that share this wave's item
    // rows, 32 each, so a 64-column block is two of them and a 128-column block all four.
    // Their row amax meet in the weight tile of the stage of the unit's last step, which no
    // load targets until the next unit's first step; the barrier shows that every wave is
    // done reading it.
    float(*amax_buf)[ROWS] = reinterpret_cast<float(*)[ROWS]>(sh.st[(s_base + KS - 1) % kStages].w);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    float cval[NG > 0 ? NG : 1][2][4];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      float amax = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x1 = acc[h][g][i], x2 = acc[2 + h][g][i];
          cval[g][h][i] = x2 * __builtin_amdgcn_rcpf(1.0f + __expf(-x2)) * x1;
          amax = fmaxf(amax, fabsf(cval[g][h][i]));
        }
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      if (lane < 16) amax_buf[wb][c.m0 + 16 * g + lane] = amax;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int m = c.m0 + 16 * g + (lane & 15);
      const float amax = S::kQCols == 64
                             ? fmaxf(amax_buf[wb & 2][m], amax_buf[(wb & 2) + 1][m])
                             : fmaxf(fmaxf(amax_buf[0][m], amax_buf[1][m]), fmaxf(amax_buf[2][m], amax_buf[3][m]));
      const float scale = fmaxf(amax / 448.0f, 1e-12f);
      const float inv = __builtin_amdgcn_rcpf(scale);
      if (m < c.rows) {
        uint8_t* dst = p.act + (size_t)(c.r0 + m) * kInter + c.tile * 128 + 32 * wb + 4 * (lane >> 4);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<uint32_t*>(dst + 16 * h) =
              pack_fp8x4(cval[g][h][0] * inv, cval[g][h][1] * inv, cval[g][h][2] * inv, cval[g][h][3] * inv);
        // the first wave of each scale block writes the block's scale
        if ((wb & (S::kQCols / 32 - 1)) == 0 && lane < 16)
          p.act_scale[(size_t)(c.r0 + m) * S::kQBlocks + (c.tile * 128 + 32 * wb) / S::kQCols] = scale;
      }
    }
    __syncthreads();
  } else {
    // Each row's destination as the dispatch wrote it (the token, or -1 - its flat slot) and its
    // routing weight come from the unit's set-up, a unit ahead (loaded here, they cost the
    // epilogue a round trip).
    // (W32: the lane's row is c.m0 + 32g + lane%32, its 16 values four runs of 4 consecutive
    // hidden columns, 8q + 4(lane/32) .. +3 of each 32-row weight block)
    constexpr int kGRows = W32 ? 32 : 16;
    const int* dest = c.dest;
    const float* wt = c.wt;
    // every load of this wave has landed, the next unit's first two steps included, before the
    // first store
    wait_vmcnt<0>();
    if (claim != nullptr && threadIdx.x == 0) sh.next = got;
    // The lane's 4-value runs of group g: run i at hidden column h0 + col(i) of the unit's tile,
    // its values already weighted. Each group decides once where its row goes (the token's output
    // row, bf16 or fp32, or the parked fp32 row), so that a row's stores share one branch.
    constexpr int kRuns = W32 ? 8 : 4;
    const int h0 = c.tile * kTileW + 64 * wb;
    auto run_col = [&](int i) {
      return W32 ? 32 * (i >> 2) + 8 * (i & 3) + 4 * (lane >> 5) : 16 * i + 4 * (lane >> 4);
    };
    const bool bf16_out = p.out_dtype == MOE_FP8_OUT_BF16;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int m = c.m0 + kGRows * g + (lane & (kGRows - 1));
      v4f val[kRuns];
#pragma unroll
      for (int i = 0; i < kRuns; ++i) {
        if constexpr (W32) {
          const v16f& a = acc32[i >> 2][g];
          const int q = i & 3;
          val[i] = v4f{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]} * wt[g];
        } else {
          val[i] = acc[i][g] * wt[g];
        }
      }
      const int d = dest[g];
      if (m < c.rows && d >= 0 && bf16_out) {
        uint16_t* row = reinterpret_cast<uint16_t*>(p.out) + (size_t)d * kHidden + h0;
#pragma unroll
        for (int i = 0; i < kRuns; ++i)
          *reinterpret_cast<uint2*>(row + run_col(i)) = pack_bf16x4(val[i][0], val[i][1], val[i][2], val[i][3]);
      } else if (m < c.rows) {
        float* row = (d >= 0 ? reinterpret_cast<float*>(p.out) + (size_t)d * kHidden
                             : p.partial + (size_t)(-1 - d) * kHidden) + h0;
#pragma unroll
        for (int i = 0; i < kRuns; ++i) *reinterpret_cast<v4f*>(row + run_col(i)) = val[i];
      }
    }
  }
  if (G1 && claim != nullptr && threadIdx.x == 0) sh.next = got;
}

// NG (row groups of this wave's half) as a template argument: instantiations 0..kMaxNG.
template <bool G1, int ROWS, int NG = 0>
__device__ __forceinline__ void tile_body_ng(const GemmParams& p, const TileCtx<ROWS>& c, const TileCtx<ROWS>& n,
                                             bool have_n, int s_base, bool pre, TileShared<ROWS>& sh,
                                             unsigned long long* claim, unsigned long long inc) {
  constexpr int kMax = (!G1 && TileShape<ROWS>::kW32) ? TileShape<ROWS>::kMaxNG32 : TileShape<ROWS>::kMaxNG;
  if constexpr (NG < kMax) {
    if (c.ng == NG) tile_body<G1, NG, ROWS>(p, c, n, have_n, s_base, pre, sh, claim, inc);
    else tile_body_ng<G1, ROWS, NG + 1>(p, c, n, have_n, s_base, pre, sh, claim, inc);
  } else {
    tile_body<G1, NG, ROWS>(p, c, n, have_n, s_base, pre, sh, claim, inc);
  }
}

// The experts of the order the dispatch recorded (descending item rows, experts with items
// first), lane k < 32 of every wavefront holding the k-th: its first item and item count and
// the geometry of its items (expert index, first row, rows of every item but the last, rows of
// the last). Read once per launch, so that a work unit's item costs no memory round trip.
struct ExpertTable {
  int first, ne, e, r0, chunk, last;
};

__device__ __forceinline__ ExpertTable expert_table(const GemmParams& p, int n_items) {
  const int lane = threadIdx.x & 63;
  ExpertTable t;
  const int ord = lane < kExpertsLocal ? p.counters[kCtrOrder + lane] : 0;
  t.first = ord & 0xFFFF;
  t.ne = ord >> 16;
  if (t.first + t.ne > n_items) t.ne = 0;
  const int4* wi = reinterpret_cast<const int4*>(p.work_items);
  const int4 a = t.ne > 0 ? wi[t.first] : int4{0, 0, 0, 0};
  t.last = t.ne > 0 ? wi[t.first + t.ne - 1].z : 0;
  t.e = a.x;
  t.r0 = a.y;
  t.chunk = a.z;
  return t;
}

// The pointers and item of work unit u for this lane (all of it wave-uniform but the DMA
// offsets and the lane's block scales). Unit u of the expert whose items start at item `first`
// is (item first + v % items, weight tile v / items) with v = u - first * TILES.
template <bool G1, int ROWS>
__device__ __forceinline__ void unit_setup(const GemmParams& p, const ExpertTable& tab, int u, TileCtx<ROWS>& c) {
  using S = TileShape<ROWS>;
  constexpr int TILES = (G1 ? 2 * kInter : kHidden) / kTileW;
  constexpr int KS = G1 ? kHBlocks : kIBlocks;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned long long m = __ballot(lane < kExpertsLocal && tab.ne > 0 && u >= tab.first * TILES &&
                                        u < (tab.first + tab.ne) * TILES);
  // (a unit no expert holds cannot come from the lists; it would run as an empty item of
  // expert 0, tile 0, rows from 0)
  const int k = m != 0 ? __builtin_ctzll(m) : 0;
  const int ne = m != 0 ? __builtin_amdgcn_readlane(tab.ne, k) : 1;
  const int v = m != 0 ? u - __builtin_amdgcn_readlane(tab.first, k) * TILES : 0;
  const int item = v % ne;
  const int chunk = __builtin_amdgcn_readlane(tab.chunk, k);
  const int e = m != 0 ? __builtin_amdgcn_readlane(tab.e, k) : 0;
  c.r0 = m != 0 ? __builtin_amdgcn_readlane(tab.r0, k) + item * chunk : 0;
  c.rows = m == 0 ? 0 : item == ne - 1 ? __builtin_amdgcn_readlane(tab.last, k) : chunk;
  c.tile = v / ne;

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
  // activation DMA j of this wave fills tile rows 8i .. 8i+7 with i = wave + 8j (j = 2 for
  // waves 0-3 of the 160-row tile only; otherwise unused)
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int blk = min(wave + kTileWaves * j, S::kABlocks - 1);
    const int m = 8 * blk + (lane >> 3);
    const int mm = m < c.rows ? m : 0;
    const int ch = (lane & 7) ^ ((m >> 1) & 7);
    size_t row;
    if constexpr (G1) row = (size_t)p.sorted_token[c.r0 + mm] * kHidden;
    else row = (size_t)(c.r0 + mm) * kInter;
    c.asrc[j] = (G1 ? p.hidden : p.act) + row + ch * 16;
  }
  {
    // the wave's 64-row block of scales: w % 4 (128 rows; GEMM2 with two scales per K-step
    // (w / 2) % 4, half w % 2) or w - 4 (160 rows, waves 4-7), capped at the last block
    constexpr bool H2 = !G1 && S::kSHalves == 2;
    c.sblk = min(S::kThirdBlock ? max(wave - 4, 0) : (H2 ? (wave >> 1) & 3 : (wave & 3)), S::kSBlocks - 1);
    c.shalf = H2 ? (wave & 1) : 0;
    const int m = 64 * c.sblk + lane;
    const int mm = m < c.rows ? m : 0;
    if constexpr (G1) c.ssrc = p.hidden_scale + p.sorted_token[c.r0 + mm];
    else c.ssrc = p.act_scale + (size_t)(c.r0 + mm) * S::kQBlocks + c.shalf;
    c.sstride = G1 ? (size_t)p.T : (size_t)S::kSHalves;
  }
  const float* swp0;
  const float* swp1;
  if constexpr (G1) {
    swp0 = p.w13_scale + ((size_t)e * 32 + c.tile) * kHBlocks;
    swp1 = p.w13_scale + ((size_t)e * 32 + kIBlocks + c.tile) * kHBlocks;
  } else {
    swp0 = p.w2_scale + ((size_t)e * kHBlocks + (c.tile * kTileW + 64 * (wave & 3)) / 128) * kIBlocks;
    swp1 = swp0;
  }
  c.sw0_lane = swp0[lane < KS ? lane : 0];
  c.sw1_lane = swp1[lane < KS ? lane : 0];
  // the item's row groups (16 rows; 32 for the 32x32x64 GEMM2), split between the two
  // wavefront halves (half 0 takes the odd one)
  constexpr int kGRows = (!G1 && S::kW32) ? 32 : 16;
  const int groups = (c.rows + kGRows - 1) / kGRows;
  const int g0 = (groups + 1) >> 1;
  c.ng = (wave >> 2) == 0 ? g0 : groups - g0;
  c.m0 = (wave >> 2) == 0 ? 0 : kGRows * g0;
  if constexpr (!G1) {
    constexpr int kMaxG = S::kW32 ? S::kMaxNG32 : S::kMaxNG;
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) {
      const int m = c.m0 + kGRows * g + (lane & (kGRows - 1));
      const int pr = c.r0 + (m < c.rows ? m : 0);
      c.dest[g] = p.row_dest[pr];
      c.wt[g] = p.sorted_weight[pr];
    }
  }
}

// A per-XCD work list (see the top of the file). Lane k < 32 of every wavefront holds
// the k-th expert of the order the dispatch recorded: its first item, item count, first weight
// tile on this XCD and the list position of its first unit.
template <int TILES>
struct XcdList {
  int first, ne, t0, pos;
  int total;   // entries of the list (wave-uniform)

  // Work unit of list entry j; false past the end. j must be wave-uniform.
  __device__ __forceinline__ bool entry(int j, int& u) const {
    if (j >= total) return false;
    const int lane = threadIdx.x & 63;
    // the last expert that starts at or before j (experts with units come first)
    const unsigned long long m = __ballot(lane < kExpertsLocal && ne > 0 && pos <= j);
    const int k = 63 - __builtin_clzll(m);
    const int ne_k = __builtin_amdgcn_readlane(ne, k);
    const int r = j - __builtin_amdgcn_readlane(pos, k);
    const int t0k = __builtin_amdgcn_readlane(t0, k);
    const int ntx = (TILES - t0k + 7) >> 3;   // the expert's tiles on this XCD
    const int item = r / ntx;
    const int tile = t0k + 8 * (r - item * ntx);
    u = __builtin_amdgcn_readlane(first, k) * TILES + tile * ne_k + item;
    return true;
  }
};

template <int TILES>
__device__ __forceinline__ XcdList<TILES> xcd_list(const ExpertTable& tab, int x) {
  XcdList<TILES> l;
  const int lane = threadIdx.x & 63;
  l.first = tab.first;
  l.ne = tab.ne;
  l.t0 = (x - 4 * (lane & 1)) & 7;
  const int len = ((TILES - l.t0 + 7) >> 3) * l.ne;
  int incl = len;
#pragma unroll
  for (int off = 1; off < kExpertsLocal; off <<= 1) {
    const int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  l.pos = incl - len;
  l.total = __builtin_amdgcn_readfirstlane(__shfl(incl, kExpertsLocal - 1));
  return l;
}

// GEMM2 with 160-row items: XCD v owns a contiguous run of the tile-major unit numbering (all
// items of one weight tile consecutive), [cut v, cut v+1). Cut v is the unit where the
// estimated work of the units before it reaches v/8 of the launch's, rounded down to a weight-
// tile boundary (cut 8: the end); a unit's estimate is its item rows plus kUnitFixedRows. Lane
// v < 8 of every wavefront holds run v. The items sharing a weight tile run together on one XCD
// and reuse the tile from its L2.
struct RangeSet {
  int begin, total;
  __device__ __forceinline__ int begin_of(int v) const { return __builtin_amdgcn_readlane(begin, v); }
  __device__ __forceinline__ int total_of(int v) const { return __builtin_amdgcn_readlane(total, v); }
};

// One XCD's run as a list: entry j is unit begin + j.
struct RangeList {
  int begin, total;
  __device__ __forceinline__ bool entry(int j, int& u) const {
    if (j >= total) return false;
    u = begin + j;
    return true;
  }
};

// Estimated fixed cost of a GEMM2 unit with 160-row items, in item rows: streaming its
// 256 x 2048 weight tile (units took 15.5 us + 0.078 us per item row at T=8192 and
// 16.6 + 0.05 on the skewed T=4096 batch). With the stealing the estimate matters little:
// 128 and 512 measured within 2 us of 256 on both batches.
constexpr int kUnitFixedRows = 256;

// The runs from the expert table (exact integer sums, so that the experts' ranges of the work
// tile it; every work-group computes the same cuts).
template <int TILES>
__device__ __forceinline__ RangeSet range_set(const ExpertTable& tab, int n_items) {
  const int lane = threadIdx.x & 63;
  const bool has = lane < kExpertsLocal && tab.ne > 0;
  const int rows = has ? (tab.ne - 1) * tab.chunk + tab.last : 0;
  const long long per_tile = has ? (long long)kUnitFixedRows * tab.ne + rows : 0;
  const long long work = per_tile * TILES;
  // the work of the experts whose items come before this one's, and of all
  long long before = 0, total = 0;
  for (int k = 0; k < kExpertsLocal; ++k) {
    const int fk = __builtin_amdgcn_readlane(tab.first, k);
    const long long wk = ((long long)__builtin_amdgcn_readlane((int)(work >> 32), k) << 32) |
                         (uint32_t)__builtin_amdgcn_readlane((int)work, k);
    total += wk;
    before += fk < tab.first ? wk : 0;
  }
  int cut = n_items * TILES;
  for (int v = 0; v < 8; ++v) {
    const long long target = (total * v) >> 3;
    const unsigned long long m = __ballot(has && before <= target && target < before + work);
    if (m != 0) {
      const int k = __builtin_ctzll(m);
      const long long off = target - __shfl(before, k);
      const long long pt = __shfl(per_tile, k);
      // floor(off / pt) < TILES: a float quotient, then corrected exactly
      int t = min((int)((float)off / (float)pt), TILES - 1);
      while (t > 0 && (long long)t * pt > off) --t;
      while (t < TILES - 1 && (long long)(t + 1) * pt <= off) ++t;
      const int u = __builtin_amdgcn_readlane(tab.first, k) * TILES + t * __builtin_amdgcn_readlane(tab.ne, k);
      if (lane == v) cut = u;
    } else if (lane == v) {
      cut = v == 0 ? 0 : n_items * TILES;
    }
  }
  // every run stays inside [0, units)
  cut = min(max(cut, 0), n_items * TILES);
  RangeSet r;
  r.begin = cut;
  r.total = max(__shfl_down(cut, 1) - cut, 0);
  return r;
}

// The claim counters: one 64-bit counter per XCD and kernel, whose low half counts the claims
// of the XCD's own work-groups on its list (from the front, after the 1 (GEMM1) or 2 (GEMM2)
// entries per work-group handed out up front) and whose high half counts the units other
// XCDs' work-groups took from the back of its run. Every claim adds to one half and sees both:
// a claim is good while pre + front + back < the list's length, so the front and back claims
// never meet, and one that fails marks the list used up for good.
struct Claim {
  int front, back;
};
__device__ __forceinline__ Claim claim_of(unsigned long long o) {
  return Claim{(int)__builtin_amdgcn_readfirstlane((uint32_t)o), (int)__builtin_amdgcn_readfirstlane((uint32_t)(o >> 32))};
}

template <bool G1, int ROWS>
__global__ __launch_bounds__(kTileWaves * 64, 1) void gemm_tile_kernel(GemmParams p) {
  constexpr int TILES = (G1 ? 2 * kInter : kHidden) / kTileW;
  constexpr int KS = G1 ? kHBlocks : kIBlocks;
  // GEMM2 with 160-row items: work-groups whose XCD's run is used up take units from the
  // back of other XCDs' runs
  constexpr bool kSteal = !G1 && ROWS == kTileItemRowsLarge;
  __shared__ __attribute__((aligned(1024))) TileShared<ROWS> sh;

  const int n_items = min(p.counters[kCtrItems], p.max_items);
  // XCD x = blockIdx.x % 8 (the grid is a multiple of 8): a work-group starts on list entry
  // blockIdx.x / 8 (GEMM2: and reserves blockIdx.x / 8 + per_xcd) and takes each later one
  // with a claim on the XCD's counter (restarted after the launch), offset by the entries
  // handed out up front. All waves of a work-group see the same entries, so all leave together.
  const int x = blockIdx.x & 7;
  const int lane = threadIdx.x & 63;
  const int per_xcd = gridDim.x >> 3;
  const int pre = (G1 ? 1 : 2) * per_xcd;
  unsigned long long* const claims = reinterpret_cast<unsigned long long*>(p.counters + kCtrClaim) + (G1 ? 0 : 8);
  const ExpertTable tab = expert_table(p, n_items);
  auto run_list = [&](const auto& list, const RangeSet& ranges) __attribute__((always_inline)) {
    int src = x;   // the XCD whose counter the work-group claims on (the own one: its front)
    // a unit from the back of another XCD's run, the one with the most units left by a read
    // of all eight counters (wavefront 0 claims, the work-group reads the result); false once
    // every run is used up. A claim that fails leaves its run used up, so this takes at most
    // eight claims.
    auto steal = [&](int& u) __attribute__((always_inline)) -> bool {
      if constexpr (!kSteal) {
        return false;
      } else {
        if (threadIdx.x < 64) {
          int got = -1, from = x;
          for (int attempt = 0; attempt < 8; ++attempt) {
            const unsigned long long o =
                lane < 8 ? __hip_atomic_load(claims + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
            const int left = lane < 8 && lane != x
                                 ? ranges.total - pre - (int)(uint32_t)o - (int)(uint32_t)(o >> 32) : 0;
            int v = -1, most = 0;
            for (int k = 0; k < 8; ++k) {
              const int lk = __builtin_amdgcn_readlane(left, k);
              if (lk > most) {
                most = lk;
                v = k;
              }
            }
            if (v < 0) break;
            unsigned long long c = 0;
            if (lane == 0) c = atomicAdd(claims + v, 1ull << 32);
            const Claim cl = claim_of(c);
            const int tv = ranges.total_of(v);
            if (pre + cl.front + cl.back < tv) {
              got = ranges.begin_of(v) + tv - 1 - cl.back;
              from = v;
              break;
            }
          }
          if (lane == 0) {
            sh.stolen = got;
            sh.steal_from = from;
          }
        }
        wait_lgkmcnt0();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        u = __builtin_amdgcn_readfirstlane(sh.stolen);
        src = __builtin_amdgcn_readfirstlane(sh.steal_from);
        return u >= 0;
      }
    };
    // the unit of the claim made during the last unit (or a stolen one)
    auto claimed = [&](int& u) __attribute__((always_inline)) -> bool {
      const Claim cl = claim_of(sh.next);
      if (src == x) {
        if (pre + cl.front + cl.back < list.total) return list.entry(pre + cl.front, u);
      } else {
        const int tv = ranges.total_of(src);
        if (pre + cl.front + cl.back < tv) {
          u = ranges.begin_of(src) + tv - 1 - cl.back;
          return true;
        }
      }
      return steal(u);
    };
    int u;
    bool have_c = list.entry(blockIdx.x >> 3, u);
    if (!have_c) have_c = steal(u);
    if (have_c) {
      TileCtx<ROWS> c, n;
      unit_setup<G1, ROWS>(p, tab, u, c);
      bool have_n = false;
      if constexpr (!G1) {
        have_n = list.entry(per_xcd + (blockIdx.x >> 3), u);
        if (!have_n) have_n = steal(u);
      }
      if (have_n) unit_setup<G1, ROWS>(p, tab, u, n);
      else n = c;
      int s_base = 0;
      bool pre_loaded = false;
      for (;;) {
        // GEMM2 claims the entry after the reserved one only while there is one
        const bool claim_now = G1 || have_n;
        tile_body_ng<G1, ROWS>(p, c, n, have_n, s_base, pre_loaded, sh, claim_now ? claims + src : nullptr,
                               src == x ? 1ull : 1ull << 32);
        // publishes sh.next (LDS); the unit's global stores may still be in flight
        wait_lgkmcnt0();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if constexpr (G1) {
          if (!claimed(u)) break;
          unit_setup<G1, ROWS>(p, tab, u, c);
        } else {
          if (!have_n) break;
          c = n;
          have_n = claimed(u);
          if (have_n) unit_setup<G1, ROWS>(p, tab, u, n);
          else n = c;
          pre_loaded = true;
        }
        s_base = (s_base + KS) % kStages;
      }
    }
    // The last work-group of the grid to leave restarts the claim counters, so that the next
    // launch finds them at zero: every other work-group's last claim has returned before it
    // counted itself out.
    if (threadIdx.x == 0) {
      int32_t* left = p.counters + kCtrLeft + (G1 ? 0 : 1);
      if (atomicAdd(left, 1) == (int)gridDim.x - 1) {
        for (int v = 0; v < 8; ++v) atomicExch(claims + v, 0ull);
        atomicExch(left, 0);
      }
    }
  };
  if constexpr (kSteal) {
    const RangeSet ranges = range_set<TILES>(tab, n_items);
    run_list(RangeList{ranges.begin_of(x), ranges.total_of(x)}, ranges);
  } else {
    run_list(xcd_list<TILES>(tab, x), RangeSet{0, 0});
  }
}

// CU count per device (an atomic: concurrent first calls store the same value)
int num_cus_tile() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (!n) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <bool G1, int ROWS>
hipError_t launch_tile(const GemmParams& p, hipStream_t s) {
  const int tiles = (G1 ? 2 * kInter : kHidden) / kTileW;
  const int max_units = p.max_items * tiles;
  int grid = (num_cus_tile() + 7) & ~7;
  const int cap = ((max_units + 7) / 8) * 8;
  if (grid > cap) grid = cap;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_tile_kernel<G1, ROWS>), dim3(grid), dim3(kTileWaves * 64), 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm1_tile(const GemmParams& p, int rows_per_item, hipStream_t s) {
  return rows_per_item > kTileItemRowsMid ? launch_tile<true, kTileItemRowsLarge>(p, s)
                                          : launch_tile<true, kTileItemRowsMid>(p, s);
}
hipError_t launch_gemm2_tile(const GemmParams& p, int rows_per_item, hipStream_t s) {
  return rows_per_item > kTileItemRowsMid ? launch_tile<false, kTileItemRowsLarge>(p, s)
                                          : launch_tile<false, kTileItemRowsMid>(p, s);
}

}  // namespace moe
