// Decode-regime grouped fp8 block-scale GEMMs (gfx950 MFMA), the requantisation pass and
// the per-token combine of the MoE layer.
//
// Work item = (local expert e, a run of <= 32 consecutive rows of e's bucket in the sorted
// assignment order). In this regime the layer streams the weights of the touched experts
// once from HBM, so the work is cut per WAVEFRONT, not per work-group: a work unit is
// (item, weight slice of one wavefront), and the units are dealt round-robin over the
// work-groups, so that every CU streams about the same number of bytes:
//   GEMM1: slice = 16 SwiGLU columns = 16 gate rows + the matching 16 up rows of W13[e]
//          (128 slices); the epilogue writes C = silu(X2) * X1 in fp32 (kernel.py:126-129),
//          and requant_kernel turns each row's 64-column blocks into e4m3 with
//          scale = max(amax/448, 1e-12) (kernel.py:131-135, the reference's 1x64 blocks).
//   GEMM2: slice = 64 hidden rows of W2[e] (112 slices); each 128-wide K-step carries two
//          activation scales, one per 64-column half (one MFMA per half, the other half's
//          activation bytes zeroed); v = acc * routing weight
//          (kernel.py:236-237); a token with one local assignment gets v written straight
//          to its output row, the others park v in `partial` by flat slot for
//          combine_kernel (the reference adds with fp32 atomics, kernel.py:246-250).
//          Up to 64 tokens GEMM2 and the combine are one kernel instead, gemm2_slice_kernel
//          (below): a work-group per 28 hidden rows across all items, with the tokens'
//          weighted sums kept in LDS.
// A wavefront streams its weight rows and the item's activation rows into a register ring
// (the next K-step in flight while the current one computes); GEMM1's and the slice kernel's
// row-major weights go through a wavefront-private LDS ring instead (stream_accumulate_g1_lds,
// gemm2_slice_kernel). Every K-step is exactly one 128x128 scale block:
// one v_mfma_f32_16x16x128_f8f6f4 per fragment pair, then acc += mfma * (s_act * s_w) in
// fp32 (kernel.py:123-124 and :234).
//
// K-byte permutation: inside each 128-byte K block, lane group g = lane/16 holds bytes
// [16g, 16g+16) and [64+16g, 64+16g+16) of its row (weights and activations alike, so the
// dot products are unchanged). Each 16-byte load instruction of a wavefront then reads
// whole 64-byte segments of 16 rows.
#include <atomic>
#include <type_traits>

#include "moe_internal.h"
#include "moe_device.h"

namespace moe {

namespace {

constexpr int kG1 = 1;
constexpr int kG2 = 2;
constexpr int kStreamWaves = 4;                      // wavefronts per work-group

// Per kind: K-steps, weight fragments (16 rows each) per work unit, work units per item
// and depth of the register ring.
//   GEMM1: a unit is 16 SwiGLU columns = their 16 gate rows + 16 up rows (2 fragments).
//   GEMM2: a unit is 64 hidden rows (4 fragments).
// Both use a 2-slot ring (one K-step in flight per wavefront besides the one consumed; GEMM1
// 96 registers with the accumulators, GEMM2 136; batches of up to 8 tokens, whose few units
// leave most wavefront slots empty, stream GEMM1's packed copy through 4 or 6 slots, see
// gemm1_stream_dispatch_kernel), so that at decode sizes every unit has its own
// wavefront and the grid drains in one round. The whole chip then keeps ~15 MB of weight loads
// in flight; a plain HBM read peaks at 6-8 MB in flight and slows beyond. Measured at T=64:
// GEMM1 117 -> 109 us and GEMM2 64 -> 57 us against 4-slot rings and 32-row GEMM2 units; GEMM1
// with 2 slots against 3: bit-identical, 1 us faster at T=16 and T=64, 1.5-3.6 us at T=96-256;
// capping the resident work-groups to cut the loads in flight further (2 or 3 per CU) was
// slower (T=64 GEMM1 110.8 / 108.6 against 105.8 us). GEMM1 units of 32 columns (4
// fragments sharing one activation fragment per K-step, half as many units) were bit-identical
// and slower: T=64 110.3 against 105.5 us, T=16 55.6 against 54.3.
// Requantising GEMM1's fp32 rows inside GEMM2 instead of in requant_kernel was measured
// and is slower (T=64: GEMM2 + combine 68 -> 80 us): the per-element IEEE divisions, four
// times the activation bytes and fewer resident wavefronts cost more than the launch.
// Columns per requantisation scale of the GEMM1 output on the streaming path: the
// reference's 1x64 block (kernel.py:131-135); GEMM2 then applies two activation scales per
// 128-wide K block.
constexpr int kQuantCols = 64;
constexpr int kQuantBlocks = kInter / kQuantCols;    // 32 per row

template <int KIND>
struct StreamShape;
template <>
struct StreamShape<kG1> {
  static constexpr int kSteps = kHBlocks;   // K = 7168
  static constexpr int kFrags = 2;
  static constexpr int kSlices = kInter / 16;
  static constexpr int kRing = 2;
};
template <>
struct StreamShape<kG2> {
  static constexpr int kSteps = kIBlocks;   // K = 2048
  static constexpr int kFrags = 4;
  static constexpr int kSlices = kHidden / (16 * kFrags);
  static constexpr int kRing = 2;
};

// One MFMA operand fragment: bytes [16g, 16g+16) and [64+16g, +16) of a 128-byte K block
// (p already points at row + 16g).
__device__ __forceinline__ v8i load_frag(const uint8_t* p) {
  const v4i lo = *reinterpret_cast<const v4i*>(p);
  const v4i hi = *reinterpret_cast<const v4i*>(p + 64);
  return join(lo, hi);
}

// The same fragment from the packed copy of the weights (moe_fp8_pack_weights), where each
// lane's 32 bytes of a K-step are contiguous (p already points at the lane's 32 bytes).
__device__ __forceinline__ v8i load_frag_packed(const uint8_t* p) {
  const v4i lo = *reinterpret_cast<const v4i*>(p);
  const v4i hi = *reinterpret_cast<const v4i*>(p + 16);
  return join(lo, hi);
}

// Packed weights (decode kernels): W13 in blocks [expert][16-column slice][K-step] of 4096 bytes,
// the gate fragment then the up fragment; W2 in blocks [expert][16 hidden rows][K-step] of 2048
// bytes. A fragment is 64 lanes x 32 bytes in the order load_frag gives them.
constexpr size_t kPackedFrag = 64 * 32;
constexpr size_t kPackedW13Bytes = (size_t)kExpertsLocal * 2 * kInter * kHidden;

// sa: the activation scale of the lane's row for the K-step: GEMM1 one (1x128 hidden
// scales), GEMM2 two (the 1x64 scales of the K-step's two halves).
template <int NF, int NG, typename SA>
struct StreamStage {
  v8i w[NF];
  v8i a[NG];
  SA sa[NG];
};

// The accumulators of one work unit for an item of NG row groups (NG <= 2). Every K-step
// has the same shape: loads past the last step repeat the last step (cache-hot) into ring
// slots that are never read, and the weight block scales come from lane registers through
// readlane, so the loop holds no branches and the compiler's waits cover exactly the step
// being consumed. Lane l ends with rows 4*(l/16)+i of each weight fragment against row
// l%16 of each row group.
// With PACKED the weights come from the packed copy. RING > 0 overrides the ring depth of the
// kind (StreamShape::kRing).
template <int KIND, int NG, bool PACKED = false, int RING = 0>
__device__ __forceinline__ void stream_accumulate(const GemmParams& p, int e, int r0, int rows, int slice,
                                                  int lane, const int32_t* row_token,
                                                  v4f (&acc)[StreamShape<KIND>::kFrags][NG]) {
  using S = StreamShape<KIND>;
  constexpr int KS = S::kSteps;
  constexpr int NF = S::kFrags;
  constexpr int NB = RING > 0 ? RING : S::kRing;
  constexpr int KMAIN = KS - KS % NB;   // steps of the ring-unrolled main loop
  using SA = typename std::conditional<KIND == kG1, float, float2>::type;
  using Stage = StreamStage<NF, NG, SA>;

  // weight fragments and their block-scale rows; lane k of sw_lane[f] holds the scale of
  // K-step k
  const uint8_t* wf[NF];
  float sw_lane[NF];
  if constexpr (KIND == kG1) {
    const int row = slice * 16 + (lane & 15);                 // gate row; up row = + I
    if constexpr (PACKED) {
      wf[0] = p.w13 + ((size_t)e * S::kSlices + slice) * KS * 2 * kPackedFrag + lane * 32;
      wf[1] = wf[0] + kPackedFrag;
    } else {
      wf[0] = p.w13 + ((size_t)e * 2 * kInter + row) * kHidden + (lane >> 4) * 16;
      wf[1] = wf[0] + (size_t)kInter * kHidden;
    }
    sw_lane[0] = p.w13_scale[((size_t)e * 32 + slice / 8) * kHBlocks + (lane < KS ? lane : 0)];
    sw_lane[1] = p.w13_scale[((size_t)e * 32 + kIBlocks + slice / 8) * kHBlocks + (lane < KS ? lane : 0)];
  } else {
    const int row0 = slice * 16 * NF;                         // fragments at row0 + 16f
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if constexpr (PACKED)
        wf[f] = p.w2 + (((size_t)e * (kHidden / 16) + row0 / 16 + f) * KS) * kPackedFrag + lane * 32;
      else
        wf[f] = p.w2 + ((size_t)e * kHidden + row0 + 16 * f + (lane & 15)) * kInter + (lane >> 4) * 16;
    }
    const float sw = p.w2_scale[((size_t)e * kHBlocks + row0 / 128) * kIBlocks + (lane < KS ? lane : 0)];
#pragma unroll
    for (int f = 0; f < NF; ++f) sw_lane[f] = sw;
  }

  // one K-step further along a weight fragment
  // (packed W13 interleaves the gate and up fragments of a K-step)
  constexpr size_t kWStep = PACKED ? (KIND == kG1 ? 2 : 1) * kPackedFrag : 128;
  auto wload = [&](const uint8_t* q) { return PACKED ? load_frag_packed(q) : load_frag(q); };
  Stage ring[NB];
  // the weight loads of the first steps go out before the activation addresses are known
  // (GEMM1 reads them from sorted_token, one more memory round trip)
#pragma unroll
  for (int s = 0; s < NB - 1; ++s)
#pragma unroll
    for (int f = 0; f < NF; ++f) ring[s].w[f] = wload(wf[f] + s * kWStep);

  // activation rows of this lane's column in each 16-row group (rows past the item's end
  // read its first row; their results are never stored)
  const uint8_t* ap[NG];
  const float* sap[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int m = g * 16 + (lane & 15);
    const int mm = m < rows ? m : 0;
    if constexpr (KIND == kG1) {
      const int tok = row_token[r0 + mm];
      ap[g] = p.hidden + (size_t)tok * kHidden + (lane >> 4) * 16;
      sap[g] = p.hidden_scale + tok;
    } else {
      ap[g] = p.act + (size_t)(r0 + mm) * kInter + (lane >> 4) * 16;
      sap[g] = p.act_scale + (size_t)(r0 + mm) * kQuantBlocks;
    }
  }

  auto issue_a = [&](int k, Stage& st) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      st.a[g] = load_frag(ap[g] + k * 128);
      if constexpr (KIND == kG1) st.sa[g] = sap[g][(size_t)k * p.T];   // hidden scales [56, T]
      else st.sa[g] = *reinterpret_cast<const float2*>(sap[g] + 2 * k);
    }
  };
  auto issue = [&](int k, Stage& st) {
#pragma unroll
    for (int f = 0; f < NF; ++f) st.w[f] = wload(wf[f] + k * kWStep);
    issue_a(k, st);
  };
#pragma unroll
  for (int s = 0; s < NB - 1; ++s) issue_a(s, ring[s]);

#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[f][g] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  // step k: refill the slot step k-1 used with step k+NB-1, then consume slot u = k % NB
  auto step = [&](int k, int u) {
    issue(min(k + NB - 1, KS - 1), ring[(u + NB - 1) % NB]);
    // keep each step's loads ahead of its math (the scheduler would otherwise pull later
    // steps' MFMAs above these loads and shrink the ring to one step in flight)
    __builtin_amdgcn_sched_barrier(0);
    const Stage& st = ring[u];
    float sc[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) sc[f] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw_lane[f]), k));
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if constexpr (KIND == kG1) {
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const v4f d = mfma16x16x128_fp8(st.w[f], st.a[g], zero);
          acc[f][g] += d * (st.sa[g] * sc[f]);
        }
      } else {
        // the two 64-column halves of the K-step (lanes hold bytes [16j, 16j+16) of the first
        // half in a[0..3] and of the second in a[4..7]), each with its own scale
        const v4i kZero4 = {0, 0, 0, 0};
        const v8i a_lo = join(lo_half(st.a[g]), kZero4);
        const v8i a_hi = join(kZero4, hi_half(st.a[g]));
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const v4f d_lo = mfma16x16x128_fp8(st.w[f], a_lo, zero);
          const v4f d_hi = mfma16x16x128_fp8(st.w[f], a_hi, zero);
          acc[f][g] += d_lo * (st.sa[g].x * sc[f]);
          acc[f][g] += d_hi * (st.sa[g].y * sc[f]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma nounroll
  for (int k0 = 0; k0 < KMAIN; k0 += NB) {
#pragma unroll
    for (int u = 0; u < NB; ++u) step(k0 + u, u);
  }
#pragma unroll
  for (int u = 0; u < KS - KMAIN; ++u) step(KMAIN + u, u);
}

// Row-major W13 through a wavefront-private LDS ring (GEMM1 units on the caller's row-major
// weights). A 16-lane pass of a row-major fragment load touches 16 cache lines (one 16-byte
// piece of each of 16 rows), four times the lines of a pass over the packed copy, and with
// every wavefront slot streaming the CU's address path is what limits the rate. Here each
// global_load_lds instruction moves 8 whole 128-byte rows (a 16-lane pass covers 2 lines)
// and ds_read_b128 gathers the MFMA fragments from the ring. A unit's 32 weight rows of a
// K-step (the 16 gate rows, then the 16 up rows) are 4 KB, 4 DMA instructions; chunk c of
// row m sits at m * 128 + 16 * (c ^ ((m >> 1) & 7)), so that the 16 rows of a ds_read_b128
// pass fall in distinct bank groups. The activation fragment and its scale still come
// straight into registers (they are L2-resident after the first touch).
constexpr int kG1LdsRows = 32;
constexpr int kG1LdsStep = kG1LdsRows * 128;                   // bytes per K-step and wavefront
constexpr int kG1LdsDma = kG1LdsRows / 8;                      // DMA instructions per K-step

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ int lds_swz(int m, int c) { return m * 128 + ((c ^ ((m >> 1) & 7)) << 4); }

// vmcnt(n) with expcnt and lgkmcnt left unconstrained (gfx9 s_waitcnt encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(N | (7 << 4) | (15 << 8));
}

template <int NG>
__device__ __forceinline__ void stream_accumulate_g1_lds(const GemmParams& p, int e, int r0, int rows, int slice,
                                                         int lane, const int32_t* row_token, uint8_t* ring,
                                                         v4f (&acc)[2][NG]) {
  using S = StreamShape<kG1>;
  constexpr int KS = S::kSteps;
  constexpr int NB = S::kRing;
  constexpr int KMAIN = KS - KS % NB;
  // VMEM instructions of one K-step, in issue order: the weight DMAs, then per row group the
  // activation fragment (two 16-byte loads) and its scale
  constexpr int kOps = kG1LdsDma + 3 * NG;
  static_assert(kOps < 16, "vmcnt immediate");

  // lane's DMA source of instruction j at K-step 0: ring row 8j + lane/8 (gate rows 0-15,
  // up rows 16-31), the logical chunk stored at physical chunk lane%8
  uint32_t woff[kG1LdsDma];
#pragma unroll
  for (int j = 0; j < kG1LdsDma; ++j) {
    const int r = 8 * j + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const size_t grow = (size_t)e * 2 * kInter + (r < 16 ? slice * 16 + r : kInter + slice * 16 + r - 16);
    woff[j] = (uint32_t)(grow * kHidden + c * 16);
  }
  float sw_lane[2];
  sw_lane[0] = p.w13_scale[((size_t)e * 32 + slice / 8) * kHBlocks + (lane < KS ? lane : 0)];
  sw_lane[1] = p.w13_scale[((size_t)e * 32 + kIBlocks + slice / 8) * kHBlocks + (lane < KS ? lane : 0)];

  auto issue_w = [&](int k, int s) {
    uint8_t* dst = ring + s * kG1LdsStep;
#pragma unroll
    for (int j = 0; j < kG1LdsDma; ++j)
      __builtin_amdgcn_global_load_lds(p.w13 + woff[j] + k * 128, (lds_void_t*)(dst + j * 1024), 16, 0, 0);
  };
  // the first steps' weight DMAs go out before the activation addresses are known
#pragma unroll
  for (int s = 0; s < NB - 1; ++s) issue_w(s, s);

  const uint8_t* ap[NG];
  const float* sap[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int m = g * 16 + (lane & 15);
    const int mm = m < rows ? m : 0;
    const int tok = row_token[r0 + mm];
    ap[g] = p.hidden + (size_t)tok * kHidden + (lane >> 4) * 16;
    sap[g] = p.hidden_scale + tok;
  }
  struct Act {
    v8i a[NG];
    float sa[NG];
  };
  auto issue_a = [&](int k, Act& st) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      st.a[g] = load_frag(ap[g] + k * 128);
      st.sa[g] = sap[g][(size_t)k * p.T];   // hidden scales [56, T]
    }
  };
  Act ring_a[NB];
#pragma unroll
  for (int s = 0; s < NB - 1; ++s) issue_a(s, ring_a[s]);

#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[f][g] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  auto step = [&](int k, int u) {
    const int kn = min(k + NB - 1, KS - 1);
    const int sn = (u + NB - 1) % NB;
    issue_w(kn, sn);
    issue_a(kn, ring_a[sn]);
    __builtin_amdgcn_sched_barrier(0);
    // step k's loads have landed once only step kn's are in flight
    wait_vm<kOps>();
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* st = ring + u * kG1LdsStep;
    v8i wf[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const uint8_t* b = st + f * 16 * 128;
      wf[f] = join(*reinterpret_cast<const v4i*>(b + lds_swz(lane & 15, lane >> 4)),
                   *reinterpret_cast<const v4i*>(b + lds_swz(lane & 15, 4 + (lane >> 4))));
    }
    const Act& a = ring_a[u];
    float sc[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) sc[f] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sw_lane[f]), k));
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const v4f d = mfma16x16x128_fp8(wf[f], a.a[g], zero);
        acc[f][g] += d * (a.sa[g] * sc[f]);
      }
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma nounroll
  for (int k0 = 0; k0 < KMAIN; k0 += NB) {
#pragma unroll
    for (int u = 0; u < NB; ++u) step(k0 + u, u);
  }
#pragma unroll
  for (int u = 0; u < KS - KMAIN; ++u) step(KMAIN + u, u);
  // the last steps reloaded the last K-step into a slot nobody reads: let those DMAs land
  // before the ring is refilled by the next unit
  wait_vm<0>();
}

// SwiGLU of a GEMM1 unit's accumulators for row group g: silu(X2) * X1 (kernel.py:126-129).
__device__ __forceinline__ v4f swiglu4(const v4f& x1, const v4f& x2) {
  v4f c;
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = (x2[i] / (1.0f + __expf(-x2[i]))) * x1[i];
  return c;
}

// One work unit with its epilogue: GEMM1 writes fp32 SwiGLU rows for requant_kernel; GEMM2
// writes or parks the weighted rows.
// GEMM1 on row-major weights streams them through the wavefront's LDS ring `ring`
// (kNB * kG1LdsStep bytes); the other instances do not use it.
template <int KIND, int NG, bool PACKED = false, int RING = 0>
__device__ __forceinline__ void stream_unit(const GemmParams& p, int e, int r0, int rows, int slice, int lane,
                                            const int32_t* row_token, uint8_t* ring) {
  constexpr int NF = StreamShape<KIND>::kFrags;
  v4f acc[NF][NG];
  if constexpr (KIND == kG1 && !PACKED) stream_accumulate_g1_lds<NG>(p, e, r0, rows, slice, lane, row_token, ring, acc);
  else stream_accumulate<KIND, NG, PACKED, RING>(p, e, r0, rows, slice, lane, row_token, acc);
  // lane: column (lane & 15) of each row group, fragment rows 4*(lane>>4) + i
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int m = g * 16 + (lane & 15);
    if (m >= rows) continue;
    const int pr = r0 + m;
    if constexpr (KIND == kG1) {
      *reinterpret_cast<v4f*>(p.swiglu + (size_t)pr * kInter + slice * 16 + 4 * (lane >> 4)) =
          swiglu4(acc[0][g], acc[1][g]);
    } else {
      const int t = p.sorted_token[pr];
      const float wt = p.sorted_weight[pr];
      const bool direct = p.token_nlocal[t] == 1;
      const size_t slot = (size_t)p.sorted_slot[pr];
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const v4f v = acc[f][g] * wt;
        const int h = slice * 16 * NF + f * 16 + 4 * (lane >> 4);
        if (direct) {
          if (p.out_dtype == MOE_FP8_OUT_BF16)
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + (size_t)t * kHidden + h) =
                pack_bf16x4(v[0], v[1], v[2], v[3]);
          else
            *reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.out) + (size_t)t * kHidden + h) = v;
        } else {
          *reinterpret_cast<v4f*>(p.partial + slot * kHidden + h) = v;
        }
      }
    }
  }
}

// The work units of n_items items (item list and GEMM1's bucket-row -> token map in the
// workspace, or in LDS for the fused dispatch below).
template <int KIND, int MAXNG, bool PACKED = false, int RING = 0>
__device__ __forceinline__ void stream_units(const GemmParams& p, int n_items, const int4* items,
                                             const int32_t* row_token, uint8_t* ring) {
  constexpr int SL = StreamShape<KIND>::kSlices;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int units = n_items * SL;
  const int nwaves = gridDim.x * kStreamWaves;
  // unit u runs on wavefront (u % gridDim.x, (u / gridDim.x) % kStreamWaves): consecutive
  // units land on different work-groups, i.e. different CUs
  for (int u = wave * gridDim.x + blockIdx.x; u < units; u += nwaves) {
    const int item = u / SL, slice = u - (u / SL) * SL;
    const int4 it = items[item];
    const int e = __builtin_amdgcn_readfirstlane(it.x);
    const int r0 = __builtin_amdgcn_readfirstlane(it.y);
    const int rows = __builtin_amdgcn_readfirstlane(it.z);
    if (MAXNG == 1 || rows <= 16) stream_unit<KIND, 1, PACKED, RING>(p, e, r0, rows, slice, lane, row_token, ring);
    else stream_unit<KIND, MAXNG, PACKED, RING>(p, e, r0, rows, slice, lane, row_token, ring);
  }
}

// PACKED: p.w13 / p.w2 is the packed copy (moe_fp8_run_packed).
template <int KIND, int MAXNG, bool PACKED = false>
__global__ __launch_bounds__(kStreamWaves * 64) void gemm_stream_kernel(GemmParams p) {
  const int n_items = min(p.counters[kCtrItems], p.max_items);
  if constexpr (KIND == kG1 && !PACKED) {
    __shared__ __attribute__((aligned(1024))) uint8_t ring[kStreamWaves][StreamShape<kG1>::kRing * kG1LdsStep];
    stream_units<KIND, MAXNG, PACKED>(p, n_items, reinterpret_cast<const int4*>(p.work_items), p.sorted_token,
                                      ring[threadIdx.x >> 6]);
  } else {
    stream_units<KIND, MAXNG, PACKED>(p, n_items, reinterpret_cast<const int4*>(p.work_items), p.sorted_token,
                                      nullptr);
  }
}

// Decode batches of up to kFusedDispatchTokens tokens: GEMM1 without a dispatch launch before
// it. Every work-group rebuilds the call's dispatch from the top-k lists in LDS, the same as
// dispatch_small_kernel produces (kernel.py:252-407 builds the equivalents): per local
// expert the assignments in ascending flat slot order t*8+k (a stable sort by expert), CSR
// offsets and the work list of 16-row items. Work-group 0 also writes it to the workspace
// for the requantisation, GEMM2 and the combine, which run after this kernel. The 512 slots
// are held two per thread, slot h*256 + tid.
constexpr int kFusedSlots = kFusedDispatchTokens * kTopK;
constexpr int kFusedItemRows = 16;
constexpr int kFusedItems = kExpertsLocal + kFusedSlots / kFusedItemRows;
constexpr int kFusedHalves = kFusedSlots / (kStreamWaves * 64);
static_assert(kFusedHalves == 2, "two slots per thread");

// The row-major instance's LDS weight rings live in the same object as the dispatch (one
// __shared__ object: the compiler then keeps the ring's DMA writes apart from its reads).
template <bool RING>
struct FusedDispatch {
  uint8_t ring[RING ? kStreamWaves : 0][StreamShape<kG1>::kRing * kG1LdsStep];
  int4 items[kFusedItems];
  int32_t row_token[kFusedSlots];
  int cnt[kFusedHalves * kStreamWaves][kExpertsLocal];   // per-wavefront counts -> prefix
  int start[kExpertsLocal];
  int n_items;
};

template <bool RING>
__device__ __forceinline__ void fused_dispatch(const GemmParams& p, const RouteParams& rp, FusedDispatch<RING>& s) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const bool writer = blockIdx.x == 0;
  const int nslots = p.T * kTopK;
  const uint64_t lt = lanemask_lt();
  int le[kFusedHalves], rank[kFusedHalves];
#pragma unroll
  for (int h = 0; h < kFusedHalves; ++h) {
    const int slot = h * kStreamWaves * 64 + tid;
    const int l = (slot < nslots ? p.topk_ids[slot] : -1) - p.offset;
    le[h] = slot < nslots && l >= 0 && l < kExpertsLocal ? l : -1;
  }
  // stable rank of each slot among the wavefront's slots of its expert, per-wavefront counts:
  // one ballot per distinct local expert of the wavefront (a few at decode sizes)
#pragma unroll
  for (int h = 0; h < kFusedHalves; ++h) {
    int* cnt = s.cnt[h * kStreamWaves + wave];
    if (lane < kExpertsLocal) cnt[lane] = 0;
    rank[h] = 0;
    uint64_t todo = __ballot(le[h] >= 0);
    while (todo) {
      const int v = __builtin_amdgcn_readlane(le[h], __builtin_ctzll(todo));
      const uint64_t m = __ballot(le[h] == v);
      if (le[h] == v) rank[h] = __popcll(m & lt);
      if (lane == 0) cnt[v] = __popcll(m);
      todo &= ~m;
    }
    if (writer) {
      // the 8 slots of a token are 8 consecutive lanes
      const uint64_t m = __ballot(le[h] >= 0);
      const int slot = h * kStreamWaves * 64 + tid;
      if ((tid & 7) == 0 && slot < nslots) rp.token_nlocal[slot >> 3] = __popcll((m >> (lane & 56)) & 0xFFull);
    }
  }
  __syncthreads();
  if (tid < kExpertsLocal) {
    // lane e of wavefront 0: expert e's wavefront prefix, CSR offset and items
    const int e = tid;
    int run = 0;
#pragma unroll
    for (int q = 0; q < kFusedHalves * kStreamWaves; ++q) {
      const int v = s.cnt[q][e];
      s.cnt[q][e] = run;
      run += v;
    }
    int incl = run;
#pragma unroll
    for (int off = 1; off < kExpertsLocal; off <<= 1) {
      const int o = __shfl_up(incl, off, kExpertsLocal);
      if (e >= off) incl += o;
    }
    const int start = incl - run;
    s.start[e] = start;
    const int nch = (run + kFusedItemRows - 1) / kFusedItemRows;
    int ich = nch;
#pragma unroll
    for (int off = 1; off < kExpertsLocal; off <<= 1) {
      const int o = __shfl_up(ich, off, kExpertsLocal);
      if (e >= off) ich += o;
    }
    const int first = ich - nch;
    for (int c = 0; c < nch; ++c) {
      const int4 it = make_int4(e, start + c * kFusedItemRows, min(kFusedItemRows, run - c * kFusedItemRows),
                                first | (nch << 16));
      s.items[first + c] = it;
      if (writer) reinterpret_cast<int4*>(rp.work_items)[first + c] = it;
    }
    if (e == kExpertsLocal - 1) s.n_items = ich;
    if (writer) {
      rp.expert_count[e] = run;
      rp.expert_start[e + 1] = incl;
      if (e == 0) rp.expert_start[0] = 0;
      if (e == kExpertsLocal - 1) {
        rp.counters[kCtrAssign] = incl;
        rp.counters[kCtrItems] = ich;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < kFusedHalves; ++h) {
    if (le[h] < 0) continue;
    const int slot = h * kStreamWaves * 64 + tid;
    const int row = s.start[le[h]] + s.cnt[h * kStreamWaves + wave][le[h]] + rank[h];
    s.row_token[row] = slot >> 3;
    if (writer) {
      rp.sorted_token[row] = slot >> 3;
      rp.sorted_weight[row] = rp.topk_w[slot];
      rp.sorted_slot[row] = slot;
    }
  }
  __syncthreads();
}

// PACKED: p.w13 is the packed copy of W13 (moe_fp8_run_packed). RING: the depth of the packed
// instance's register ring (0: StreamShape<kG1>::kRing; gemm1_stream_dispatch_deep_kernel).
// Small batches take deeper rings (RING - 1 K-steps in flight per wavefront instead of one):
// they touch a few experts, so only a few hundred wavefronts stream and each one's depth sets
// the rate. Measured through the C ABI on seeded batches (two runs each, us per layer, 2 / 3 /
// 4 slots): T=1 with 2 experts 34.6 / 30.8 / 29.3, T=2 with 3 experts 41.2 / 37.5 / 35.8, T=4
// with 4 experts 45.0 / 42.1 / 42.5, T=8 with 3 experts 41.6 / 37.7 / 36.2; with 5-6 experts
// (640-768 units) within +-0.5; at T=16 (10 experts, 1280 units) 84.8 / 86.3 / 85.3, hence
// the bound of 8 tokens. 4 / 6 / 8 slots: 2 experts (256 units) 30.4 / 28.4 / 28.0 and 30.3 /
// 27.9 / 27.9, 3 experts 36.3 / 35.9 / 36.5, 5 experts 49.9 / 50.8 / 51.7: 6 slots up to 2
// tokens. Bit-identical to the 2-slot ring.
constexpr int kDeepRingTokens = 8;
constexpr int kDeepRing = 4;
constexpr int kDeeperRingTokens = 2;
constexpr int kDeeperRing = 6;

template <bool PACKED, int RING>
__device__ __forceinline__ void gemm1_stream_dispatch(const GemmParams& p, const RouteParams& rp) {
  static_assert(RING == 0 || PACKED, "the row-major instance's LDS ring waits assume StreamShape's depth");
  __shared__ __attribute__((aligned(1024))) FusedDispatch<!PACKED> s;
  fused_dispatch(p, rp, s);
  uint8_t* ring = nullptr;
  if constexpr (!PACKED) ring = s.ring[threadIdx.x >> 6];
  stream_units<kG1, 1, PACKED, RING>(p, s.n_items, s.items, s.row_token, ring);
}

template <bool PACKED>
__global__ __launch_bounds__(kStreamWaves * 64) void gemm1_stream_dispatch_kernel(GemmParams p, RouteParams rp) {
  gemm1_stream_dispatch<PACKED, 0>(p, rp);
}

// The packed instance on a RING-slot register ring (batches of up to kDeepRingTokens tokens).
template <int RING>
__global__ __launch_bounds__(kStreamWaves * 64) void gemm1_stream_dispatch_deep_kernel(GemmParams p, RouteParams rp) {
  gemm1_stream_dispatch<true, RING>(p, rp);
}

// Requantises the fp32 SwiGLU rows: per row and COLS columns, scale = max(amax/448, 1e-12)
// and q = e4m3(c / scale) (kernel.py:131-135, whose blocks are 64 columns wide). One
// work-group of 256 threads per row, 8 columns per thread, COLS/8 threads per block.
template <int COLS>
__global__ __launch_bounds__(256) void requant_kernel(GemmParams p) {
  constexpr int kThreads = COLS / 8;
  constexpr int kBlocks = kInter / COLS;
  const int nmax = p.T * kTopK;   // rows of the SwiGLU buffer
  const int tid = threadIdx.x;
  for (int r = blockIdx.x; r < nmax; r += gridDim.x) {
    // the row is loaded together with the number of rows in use (no dependent round trip)
    const v4f* src = reinterpret_cast<const v4f*>(p.swiglu + (size_t)r * kInter) + 2 * tid;
    const v4f a = src[0], b = src[1];
    if (r >= p.counters[kCtrAssign]) break;
    float amax = fmaxf(fmaxf(fmaxf(fabsf(a[0]), fabsf(a[1])), fmaxf(fabsf(a[2]), fabsf(a[3]))),
                       fmaxf(fmaxf(fabsf(b[0]), fabsf(b[1])), fmaxf(fabsf(b[2]), fabsf(b[3]))));
#pragma unroll
    for (int off = 1; off < kThreads; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float scale = fmaxf(amax / 448.0f, 1e-12f);
    uint2 q;
    q.x = pack_fp8x4(a[0] / scale, a[1] / scale, a[2] / scale, a[3] / scale);
    q.y = pack_fp8x4(b[0] / scale, b[1] / scale, b[2] / scale, b[3] / scale);
    reinterpret_cast<uint2*>(p.act + (size_t)r * kInter)[tid] = q;
    if (tid % kThreads == 0) p.act_scale[(size_t)r * kBlocks + tid / kThreads] = scale;
  }
}

// Decode batches of up to kFusedDispatchTokens tokens (16-row items): GEMM2 and the combine in
// one kernel, with no fp32 rows parked in `partial`. A work-group owns 28 hidden rows of W2
// (256 slices, one per CU: two MFMA fragments, the second's last four rows repeating its last
// row and never stored) across every work item, and its wavefront q owns K-steps
// [2q, 2q+2) of each: per item, q streams the expert's 32 x 256 weight bytes and the item's
// act rows through a register ring, scales each 128-wide block product (kernel.py:234),
// weights it by the routing weight (kernel.py:236-237) and adds it into its own LDS
// accumulator of (token, hidden row). Items come in expert order, so each token's
// contributions are added in ascending local expert order, and the rows of one token inside
// an item (a repeated expert id) in slot order; the work-group then sums its eight K parts
// in fixed order and writes the 28 columns of every token, zeros for tokens without a local
// expert (the zero-fill and finalize of kernel.py:704, 729). Deterministic, no atomics.
// 28-row slices against 32-row ones (224 work-groups, 32 CUs idle): every output element is
// computed by the same operations in the same order, and the weight stream spreads over all
// 256 CUs. A 2-slot ring against 4 (3 steps in flight): bit-identical, 240 registers instead of
// 312, T=16 GEMM2 34.0 -> 33.4 us, T=64 unchanged.
// Slice width, measured at T=64 / T=16 (GEMM2 with the requantisation before it, us): one
// fragment 78.0 / 39.8, two 63.9 / 33.7, four 101.6 / 52.6, against 68.0 / 40.0 for the
// wavefront-per-unit GEMM2 plus combine_kernel. One fragment spends a 2 KB activation
// fragment and four small loads on every 2 KB of weights; four need more registers than two
// wavefronts per SIMD allow, and one wavefront per SIMD cannot keep the matrix core busy.
// Eight wavefronts of 2 K-steps per item (two per SIMD, 180 registers) against four of 4 (one
// per SIMD, 240): GEMM2 stage 56.7-56.8 -> 55.9-56.6 us at T=64, 32.4-32.6 -> 32.0-32.2 at T=16
// (four runs each); the K parts' sum changes order, within the parity bounds.
constexpr int kSliceF = 2;                               // weight fragments per wavefront
constexpr int kSliceRows = 28;                           // hidden rows per work-group
constexpr int kSliceParts = 8;                           // wavefronts per work-group = K parts
constexpr int kSliceSteps = kIBlocks / kSliceParts;      // 2 K-steps per part and item
constexpr int kSliceRing = 2;                            // ring slots: 1 step in flight besides the one consumed
constexpr int kHiddenSlices = kHidden / kSliceRows;      // 256
static_assert(kHidden % kSliceRows == 0 && kSliceRows > 16 * (kSliceF - 1) && kSliceRows <= 16 * kSliceF,
              "slice rows");
// a lane's four output rows of a fragment are 4-aligned, so they share one 128-row W2 scale block
static_assert(kSliceRows % 4 == 0 && kBlock % 4 == 0, "scale blocks");
static_assert(kSliceSteps % kSliceRing == 0, "slot u % ring is K-step u of the item");
static_assert(kFusedItems <= 64, "one work item per lane");

struct SliceStage {
  v8i w[kSliceF];   // W2 fragments: the slice's hidden rows 16f.. x 128 K bytes
  v8i a;            // act fragment: the item's 16 rows (rows past its end repeat its first row)
  float2 sa;        // act scales of the lane's row for the two 64-column halves of the K block
  float sw[kSliceF];  // W2 block scale of the lane's four output rows of each fragment
  int tok;          // token of the lane's row
  float wt;         // routing weight of the lane's row
};

// On the row-major weights the slice's 28 W2 rows of a K-step (rows past 28 repeating the
// last) go through a wavefront-private LDS ring, 8 whole rows per global_load_lds
// instruction, as for GEMM1's row-major units; the ring and the token accumulators are one
// LDS object.
constexpr int kSliceLdsRows = 16 * kSliceF;                     // 32
constexpr int kSliceLdsStep = kSliceLdsRows * 128;              // 4 KB per K-step
constexpr int kSliceLdsDma = kSliceLdsRows / 8;                 // 4 DMA instructions

template <bool RING>
struct SliceShared {
  float acc[kSliceParts][kFusedDispatchTokens][16 * kSliceF];
  uint8_t ring[RING ? kSliceParts : 0][kSliceRing * kSliceLdsStep];
};

// PACKED: p.w2 is the packed copy of W2 (moe_fp8_run_packed).
template <bool PACKED>
__global__ __launch_bounds__(kSliceParts * 64) void gemm2_slice_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(1024))) SliceShared<!PACKED> sh;
  auto& acc_lds = sh.acc;
  const int lane = threadIdx.x & 63;
  const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m = lane & 15;
  const int T = p.T;
  const int n_items = min(p.counters[kCtrItems], min(p.max_items, kFusedItems));
  const int4 my_item = lane < n_items ? reinterpret_cast<const int4*>(p.work_items)[lane] : make_int4(0, 0, 0, 0);
  const int nsteps = n_items * kSliceSteps;
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  for (int slice = blockIdx.x; slice < kHiddenSlices; slice += gridDim.x) {
    const int h0 = slice * kSliceRows;
    float* my_acc = &acc_lds[q][0][0];
    for (int i = lane; i < T * 16 * kSliceF; i += 64) my_acc[i] = 0.f;
    if (nsteps > 0) {
      // loads of flattened step st = 4 * item + j (K-step 4q + j of the item); steps past the
      // last repeat it (cache-hot, never consumed)
      auto issue = [&](int st, SliceStage& g) {
        const int sc = min(st, nsteps - 1);
        const int it = sc / kSliceSteps;
        const int ks = q * kSliceSteps + (sc - it * kSliceSteps);
        const int e = __builtin_amdgcn_readlane(my_item.x, it);
        const int r0 = __builtin_amdgcn_readlane(my_item.y, it);
        const int rows = __builtin_amdgcn_readlane(my_item.z, it);
        const int r = r0 + (m < rows ? m : 0);
        // The small loads first. The loop over items carries the ring slot that an item's last
        // step fills with the next item's first step, and the compiler's copies of its scale
        // registers at the back edge wait for those loads: issued ahead of the fragments, they
        // leave the fragment loads in flight across the item boundary (packed weights; on the
        // row-major weights the compiler still drains the ring there). Bit-identical; T=16
        // GEMM2 stage 32.7-32.8 -> 32.3-32.5 us, T=64 about 0.3 us.
#pragma unroll
        for (int f = 0; f < kSliceF; ++f) {
          const int orow = h0 + min(16 * f + 4 * (lane >> 4), kSliceRows - 1);   // first output row
          g.sw[f] = p.w2_scale[((size_t)e * kHBlocks + orow / kBlock) * kIBlocks + ks];
        }
        g.sa = *reinterpret_cast<const float2*>(p.act_scale + (size_t)r * kQuantBlocks + 2 * ks);
        g.tok = p.sorted_token[r];
        g.wt = p.sorted_weight[r];
        if constexpr (!PACKED) {
          uint8_t* dst = sh.ring[q] + (st % kSliceRing) * kSliceLdsStep;
#pragma unroll
          for (int j = 0; j < kSliceLdsDma; ++j) {
            const int rr = 8 * j + (lane >> 3);
            const int c = (lane & 7) ^ ((rr >> 1) & 7);
            const int hr = h0 + min(rr, kSliceRows - 1);
            __builtin_amdgcn_global_load_lds(p.w2 + ((size_t)e * kHidden + hr) * kInter + ks * 128 + c * 16,
                                             (lds_void_t*)(dst + j * 1024), 16, 0, 0);
          }
        }
        if constexpr (PACKED) {
#pragma unroll
          for (int f = 0; f < kSliceF; ++f) {
            // the lane's hidden row in fragment f (rows past the slice repeat its last row)
            const int hr = h0 + 16 * f + min(m, kSliceRows - 16 * f - 1);
            g.w[f] = load_frag_packed(p.w2 + (((size_t)e * (kHidden / 16) + (hr >> 4)) * kIBlocks + ks) * kPackedFrag +
                                      ((hr & 15) + 16 * (lane >> 4)) * 32);
          }
        }
        g.a = load_frag(p.act + (size_t)r * kInter + ks * 128 + (lane >> 4) * 16);
      };
      SliceStage ring[kSliceRing];
#pragma unroll
      for (int u = 0; u < kSliceRing - 1; ++u) issue(u, ring[u]);
      v4f acc[kSliceF];
#pragma unroll
      for (int f = 0; f < kSliceF; ++f) acc[f] = zero;
#pragma nounroll
      for (int st0 = 0; st0 < nsteps; st0 += kSliceSteps) {
#pragma unroll
        for (int u = 0; u < kSliceSteps; ++u) {
          issue(st0 + u + kSliceRing - 1, ring[(u + kSliceRing - 1) % kSliceRing]);
          __builtin_amdgcn_sched_barrier(0);
          const SliceStage& g = ring[u % kSliceRing];
          v8i wf[kSliceF];
          if constexpr (PACKED) {
#pragma unroll
            for (int f = 0; f < kSliceF; ++f) wf[f] = g.w[f];
          } else {
            // step st0 + u has landed once only the loads of the step just issued are in
            // flight: 4 DMAs, 2 weight scales, the act fragment (2) and its scales, plus the
            // rows' tokens and weights when that step is an item's last (the only step whose
            // are read). The counts are exact (the compiled steps issue 9 and 11 loads): a
            // step's DMAs follow its small loads, so a larger count could leave some of them
            // in flight. Covering every load of step st0 + u here also keeps the compiler
            // from waiting on the rest itself, which it would do with vmcnt(0) while the
            // ring's DMAs are in flight.
            if (u == kSliceSteps - 2) wait_vm<kSliceLdsDma + 7>();
            else wait_vm<kSliceLdsDma + 5>();
            __builtin_amdgcn_sched_barrier(0);
            const uint8_t* b = sh.ring[q] + (u % kSliceRing) * kSliceLdsStep;
#pragma unroll
            for (int f = 0; f < kSliceF; ++f)
              wf[f] = join(*reinterpret_cast<const v4i*>(b + f * 2048 + lds_swz(m, lane >> 4)),
                           *reinterpret_cast<const v4i*>(b + f * 2048 + lds_swz(m, 4 + (lane >> 4))));
          }
          // the act fragment's two 64-column halves carry their own scales: one MFMA per
          // half, the other half's bytes zeroed (lanes hold bytes [16j, 16j+16) of the first
          // half in a[0..3] and of the second in a[4..7])
          const v4i kZero4 = {0, 0, 0, 0};
          const v8i a_lo = join(lo_half(g.a), kZero4);
          const v8i a_hi = join(kZero4, hi_half(g.a));
#pragma unroll
          for (int f = 0; f < kSliceF; ++f) {
            const float sc_lo = g.sa.x * g.sw[f], sc_hi = g.sa.y * g.sw[f];
            const v4f d_lo = mfma16x16x128_fp8(wf[f], a_lo, zero);
            const v4f d_hi = mfma16x16x128_fp8(wf[f], a_hi, zero);
            acc[f] += d_lo * sc_lo;
            acc[f] += d_hi * sc_hi;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        // end of the item: its weighted rows into this wavefront's token accumulators; when a
        // token names a local expert more than once its rows are adjacent (slot order), and
        // the first one adds the others in order, so that each accumulator has one writer
        const SliceStage& g = ring[(kSliceSteps - 1) % kSliceRing];
        const int rows = __builtin_amdgcn_readlane(my_item.z, st0 / kSliceSteps);
        const bool live = m < rows;
        // token of the row above (DPP row shift: a data-share permute here would make the
        // compiler drain the ring's loads in flight)
        const int prev = __builtin_amdgcn_update_dpp(g.tok, g.tok, 0x111, 0xf, 0xf, false);
        const bool head = live && (m == 0 || prev != g.tok);
        const bool dups = __ballot(live && !head) != 0;
#pragma unroll
        for (int f = 0; f < kSliceF; ++f) {
          v4f v = acc[f] * g.wt;
          acc[f] = zero;
          if (dups) {
            v4f tot = v;
            bool run = true;
            for (int d = 1; d < 16; ++d) {
              const int ot = __shfl(g.tok, lane + d);
              v4f ov;
#pragma unroll
              for (int i = 0; i < 4; ++i) ov[i] = __shfl(v[i], lane + d);
              run = run && m + d < rows && ot == g.tok;
              if (run) tot += ov;
            }
            v = tot;
          }
          if (head) *reinterpret_cast<v4f*>(&acc_lds[q][g.tok][16 * f + 4 * (lane >> 4)]) += v;
        }
      }
      // the last steps reloaded the last K-step into a ring slot nobody reads
      if constexpr (!PACKED) wait_vm<0>();
    }
    __syncthreads();
    // the K parts, summed in fixed order: 4 columns of one token per thread (the slice's
    // 28 columns; the accumulators' last 4 hold the repeated rows)
    constexpr int kChunks = kSliceRows / 4;
    for (int i = threadIdx.x; i < T * kChunks; i += kSliceParts * 64) {
      const int t = i / kChunks, c = 4 * (i % kChunks);
      v4f s = *reinterpret_cast<const v4f*>(&acc_lds[0][t][c]);
#pragma unroll
      for (int qq = 1; qq < kSliceParts; ++qq) s += *reinterpret_cast<const v4f*>(&acc_lds[qq][t][c]);
      const size_t o = (size_t)t * kHidden + h0 + c;
      if (p.out_dtype == MOE_FP8_OUT_BF16)
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + o) = pack_bf16x4(s[0], s[1], s[2], s[3]);
      else
        *reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.out) + o) = s;
    }
    __syncthreads();
  }
}

// Output rows of every token without exactly one local assignment: the sum of its parked
// GEMM2 rows in top-k slot order, or zeros. One wavefront per (token, 1/7 of the row): the
// token's local slots become a uniform bit mask, and each lane sums 4 columns in 4 places.
// The loads are kept in flight together: the next item's top-k ids and local count are
// fetched while the current item is summed, and the parked rows are loaded two at a time
// (the additions stay in slot order).
constexpr int kCombineChunks = 7;   // 1792 float4 per row = 7 chunks x 4 x 64 lanes

__global__ __launch_bounds__(256) void combine_kernel(GemmParams p) {
  constexpr int kVecPerRow = kHidden / 4;
  constexpr int kPerLane = kVecPerRow / kCombineChunks / 64;   // 4
  const int lane = threadIdx.x & 63;
  const int nwaves = gridDim.x * 4;
  const int items = p.T * kCombineChunks;
  int it = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (it >= items) return;
  // every lane loads (lane & 7): no divergent branch, so the loads stay in flight until used
  auto meta = [&](int item, int& id, int& nl) {
    const int t = item / kCombineChunks;
    id = p.topk_ids[t * kTopK + (lane & 7)];
    nl = p.token_nlocal[t];
  };
  int id, nl;
  meta(it, id, nl);
  while (it < items) {
    const int next = it + nwaves;
    int id_n, nl_n;
    meta(min(next, items - 1), id_n, nl_n);   // past the end: a repeat, never used
    if (__builtin_amdgcn_readfirstlane(nl) != 1) {
      const int t = it / kCombineChunks, ch = it - t * kCombineChunks;
      const int le = id - p.offset;
      uint32_t m = (uint32_t)__ballot(lane < kTopK && le >= 0 && le < kExpertsLocal);
      const int v0 = ch * kPerLane * 64 + lane;
      const v4f* rows = reinterpret_cast<const v4f*>(p.partial + (size_t)t * kTopK * kHidden) + v0;
      v4f acc[kPerLane];
#pragma unroll
      for (int u = 0; u < kPerLane; ++u) acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
      while (m) {
        const int k0 = __builtin_ctz(m);
        m &= m - 1;
        const bool two = m != 0;
        const int k1 = two ? __builtin_ctz(m) : k0;
        if (two) m &= m - 1;
        const v4f* r0 = rows + (size_t)k0 * kVecPerRow;
        const v4f* r1 = rows + (size_t)k1 * kVecPerRow;
        v4f a[kPerLane], b[kPerLane];
#pragma unroll
        for (int u = 0; u < kPerLane; ++u) {
          a[u] = r0[64 * u];
          b[u] = r1[64 * u];
        }
#pragma unroll
        for (int u = 0; u < kPerLane; ++u) {
          acc[u] += a[u];
          if (two) acc[u] += b[u];
        }
      }
#pragma unroll
      for (int u = 0; u < kPerLane; ++u) {
        const size_t h4 = (size_t)t * kVecPerRow + v0 + 64 * u;
        if (p.out_dtype == MOE_FP8_OUT_BF16)
          reinterpret_cast<uint2*>(p.out)[h4] = pack_bf16x4(acc[u][0], acc[u][1], acc[u][2], acc[u][3]);
        else
          reinterpret_cast<v4f*>(p.out)[h4] = acc[u];
      }
    }
    it = next;
    id = id_n;
    nl = nl_n;
  }
}

// Host-side caches of device facts are atomics: concurrent first calls from several host
// threads each compute the same value and store it.
int num_cus() {
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

// Work-groups of `kernel` that one CU holds at once (cached per kernel; 1 if unknown).
template <typename K>
int resident_per_cu(K kernel, std::atomic<int>& cache) {
  int n = cache.load(std::memory_order_relaxed);
  if (!n) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kStreamWaves * 64, 0) != hipSuccess || n <= 0) n = 1;
    cache.store(n, std::memory_order_relaxed);
  }
  return n;
}

// One wave of resident work-groups: every work-group starts at once, and the round-robin
// deal gives every CU the same number of units (a second, partial wave of work-groups
// would run at a fraction of the occupancy).
template <int KIND, int MAXNG, bool PACKED = false>
hipError_t launch_stream_ng(const GemmParams& p, hipStream_t s) {
  static std::atomic<int> occ{0};
  const auto kernel = gemm_stream_kernel<KIND, MAXNG, PACKED>;
  const int max_units = p.max_items * StreamShape<KIND>::kSlices;
  int grid = num_cus() * resident_per_cu(kernel, occ);
  const int cap = (max_units + kStreamWaves - 1) / kStreamWaves;
  if (grid > cap) grid = cap;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(kStreamWaves * 64), 0, s, p);
  return hipGetLastError();
}

template <int KIND>
hipError_t launch_stream(const GemmParams& p, int rows_per_item, bool packed, hipStream_t s) {
  if (rows_per_item <= 16) return packed ? launch_stream_ng<KIND, 1, true>(p, s) : launch_stream_ng<KIND, 1>(p, s);
  return packed ? launch_stream_ng<KIND, 2, true>(p, s) : launch_stream_ng<KIND, 2>(p, s);
}

// Writes the packed copy of W13 and W2: one 16-byte chunk per thread and iteration, in the
// packed order (the reads gather 16-byte pieces of rows; a one-time conversion).
__global__ __launch_bounds__(256) void pack_weights_kernel(const uint8_t* __restrict__ w13, const uint8_t* __restrict__ w2,
                                                           uint8_t* __restrict__ packed) {
  constexpr size_t kChunks13 = kPackedW13Bytes / 16;
  constexpr size_t kChunks = kChunks13 + (size_t)kExpertsLocal * kHidden * kInter / 16;
  constexpr int kSlices1 = kInter / 16;
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < kChunks; c += (size_t)gridDim.x * blockDim.x) {
    const size_t o = c * 16;   // byte offset in the packed copy
    const int half = (int)(o >> 4) & 1;
    const int lane = (int)(o >> 5) & 63;
    const int col16 = (lane >> 4) * 16 + half * 64;   // byte of the 128-byte K block
    const uint8_t* src;
    if (c < kChunks13) {
      const size_t blk = o / (2 * kPackedFrag);       // (expert, slice, K-step)
      const int f = (int)(o / kPackedFrag) & 1;       // gate, up
      const int k = (int)(blk % kHBlocks);
      const int slice = (int)((blk / kHBlocks) % kSlices1);
      const int e = (int)(blk / ((size_t)kHBlocks * kSlices1));
      const int row = f * kInter + slice * 16 + (lane & 15);
      src = w13 + ((size_t)e * 2 * kInter + row) * kHidden + k * 128 + col16;
    } else {
      const size_t o2 = o - kPackedW13Bytes;
      const size_t blk = o2 / kPackedFrag;            // (expert, 16 hidden rows, K-step)
      const int k = (int)(blk % kIBlocks);
      const int h = (int)((blk / kIBlocks) % (kHidden / 16));
      const int e = (int)(blk / ((size_t)kIBlocks * (kHidden / 16)));
      src = w2 + ((size_t)e * kHidden + h * 16 + (lane & 15)) * kInter + k * 128 + col16;
    }
    *reinterpret_cast<v4i*>(packed + o) = *reinterpret_cast<const v4i*>(src);
  }
}

}  // namespace

size_t packed_weights_bytes() { return kPackedW13Bytes + (size_t)kExpertsLocal * kHidden * kInter; }

hipError_t launch_pack_weights(const uint8_t* w13, const uint8_t* w2, uint8_t* packed, hipStream_t s) {
  hipLaunchKernelGGL(pack_weights_kernel, dim3(num_cus() * 8), dim3(256), 0, s, w13, w2, packed);
  return hipGetLastError();
}

hipError_t launch_gemm1(const GemmParams& p, int rows_per_item, bool packed, hipStream_t s) {
  if (rows_per_item > 32) return launch_gemm1_tile(p, rows_per_item, s);
  return launch_stream<kG1>(p, rows_per_item, packed, s);
}

hipError_t launch_gemm1_dispatch(const GemmParams& p, const RouteParams& rp, bool packed, hipStream_t s) {
  // one wave of resident work-groups of the instance launched (each has its own occupancy)
  static std::atomic<int> occ_rows{0}, occ_packed{0}, occ_deep{0}, occ_deeper{0};
  if (p.T <= 0 || p.T > kFusedDispatchTokens || rp.rows_per_item != kFusedItemRows) return hipErrorInvalidValue;
  const bool deeper = packed && p.T <= kDeeperRingTokens;
  const bool deep = packed && !deeper && p.T <= kDeepRingTokens;
  int grid = num_cus() * (deeper   ? resident_per_cu(gemm1_stream_dispatch_deep_kernel<kDeeperRing>, occ_deeper)
                          : deep   ? resident_per_cu(gemm1_stream_dispatch_deep_kernel<kDeepRing>, occ_deep)
                          : packed ? resident_per_cu(gemm1_stream_dispatch_kernel<true>, occ_packed)
                                   : resident_per_cu(gemm1_stream_dispatch_kernel<false>, occ_rows));
  const int cap = (kFusedItems * StreamShape<kG1>::kSlices + kStreamWaves - 1) / kStreamWaves;
  if (grid > cap) grid = cap;
  if (deeper)
    hipLaunchKernelGGL(gemm1_stream_dispatch_deep_kernel<kDeeperRing>, dim3(grid), dim3(kStreamWaves * 64), 0, s, p, rp);
  else if (deep)
    hipLaunchKernelGGL(gemm1_stream_dispatch_deep_kernel<kDeepRing>, dim3(grid), dim3(kStreamWaves * 64), 0, s, p, rp);
  else if (packed)
    hipLaunchKernelGGL(gemm1_stream_dispatch_kernel<true>, dim3(grid), dim3(kStreamWaves * 64), 0, s, p, rp);
  else
    hipLaunchKernelGGL(gemm1_stream_dispatch_kernel<false>, dim3(grid), dim3(kStreamWaves * 64), 0, s, p, rp);
  return hipGetLastError();
}

hipError_t launch_requant(const GemmParams& p, int rows_per_item, hipStream_t s) {
  if (rows_per_item > 32) return hipSuccess;   // the tile GEMM1 requantises in its epilogue
  int grid = p.T * kTopK;                      // rows of the SwiGLU buffer
  if (grid > num_cus() * 8) grid = num_cus() * 8;
  if (grid <= 0) return hipSuccess;
  static_assert(kQuantCols == 64, "the streaming path requantises per 64 columns");
  if (requant_block_for(rows_per_item) != kQuantCols) return hipErrorInvalidValue;
  hipLaunchKernelGGL(requant_kernel<kQuantCols>, dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_gemm2(const GemmParams& p, int rows_per_item, bool packed, hipStream_t s) {
  if (rows_per_item > 32) return launch_gemm2_tile(p, rows_per_item, s);
  if (rows_per_item == kFusedItemRows) {
    // up to 64 tokens: GEMM2 with the combine, one work-group per 32-row hidden slice
    if (p.T > kFusedDispatchTokens) return hipErrorInvalidValue;
    if (packed) hipLaunchKernelGGL(gemm2_slice_kernel<true>, dim3(kHiddenSlices), dim3(kSliceParts * 64), 0, s, p);
    else hipLaunchKernelGGL(gemm2_slice_kernel<false>, dim3(kHiddenSlices), dim3(kSliceParts * 64), 0, s, p);
    return hipGetLastError();
  }
  return launch_stream<kG2>(p, rows_per_item, packed, s);
}

hipError_t launch_combine(const GemmParams& p, int rows_per_item, hipStream_t s) {
  if (p.T <= 0 || rows_per_item == kFusedItemRows) return hipSuccess;   // combined in GEMM2
  // 4 (token, chunk) items per work-group at a time; up to 32 work-groups per CU (against 8:
  // GEMM2 + combine at T=8192 247-248 -> 243-244 us, unchanged at T=1024 and on the skewed
  // T=4096 batch)
  int grid = (p.T * kCombineChunks + 3) / 4;
  if (grid > num_cus() * 32) grid = num_cus() * 32;
  hipLaunchKernelGGL(combine_kernel, dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace moe
