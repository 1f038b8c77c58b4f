// Internal declarations shared by the HIP translation units of libmoe_fp8.
//
// Data layout in HBM (all row-major, contiguous):
//   caller tensors   : the contract of kernel.py:591-607 (see include/moe_fp8.h)
//   workspace arrays : moe_fp8_layout offsets; every array is 256-byte aligned.
// Kernels of one call run in this order on one stream:
//   T <= 64 (moe_fp8_run): route_wide_kernel -> gemm1_stream_dispatch_kernel (GEMM1 that
//   rebuilds the dispatch itself) -> requant_kernel -> gemm2_slice_kernel (GEMM2 and the
//   combine); otherwise
//   route_wide_kernel -> dispatch_small_kernel (T <= 256) | route_kernel -> place_kernel
//   -> GEMM1 -> [requant_kernel] -> GEMM2 -> [combine_kernel]
// where, with <= 32 rows per work item, GEMM1 is gemm_stream_kernel<1> and leaves fp32 SwiGLU
// rows for requant_kernel, and GEMM2 is gemm2_slice_kernel (16-row items, up to 64 tokens)
// or gemm_stream_kernel<2> followed by combine_kernel; with more rows both GEMMs are
// gemm_tile_kernel, GEMM1 requantises in its epilogue and combine_kernel follows GEMM2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moe_fp8.h"

namespace moe {

constexpr int kHidden = MOE_FP8_HIDDEN;        // 7168
constexpr int kInter = MOE_FP8_INTER;          // 2048
constexpr int kExpertsGlobal = MOE_FP8_EXPERTS_GLOBAL;
constexpr int kExpertsLocal = MOE_FP8_EXPERTS_LOCAL;
constexpr int kTopK = MOE_FP8_TOP_K;
constexpr int kNGroup = MOE_FP8_N_GROUP;
constexpr int kTopKGroup = MOE_FP8_TOPK_GROUP;
constexpr int kGroupSize = kExpertsGlobal / kNGroup;  // 32
constexpr int kBlock = MOE_FP8_BLOCK;          // 128
constexpr int kHBlocks = MOE_FP8_H_BLOCKS;     // 56
constexpr int kIBlocks = MOE_FP8_I_BLOCKS;     // 16

// Routing: up to kWideRouteTokens tokens one token per wavefront (4 per work-group), above
// that 16 lanes per token and 16 tokens per work-group of 4 wavefronts; the one-work-group
// dispatch of small batches uses 1024 threads.
constexpr int kWideRouteTokens = 256;
constexpr int kRouteTokensPerBlock = 16;
constexpr int kRouteThreads = 1024;
// Up to this many tokens routing and dispatch run in a single work-group (one launch).
constexpr int kSinglePassTokens = 256;
// Up to this many tokens moe_fp8_run launches routing alone, and every GEMM1 work-group
// rebuilds the dispatch in LDS (work-group 0 also writes it to the workspace).
constexpr int kFusedDispatchTokens = 64;

// Control block (workspace counters[]).
constexpr int kCtrItems = 0;    // number of GEMM work items
constexpr int kCtrAssign = 1;   // N, the number of local assignments
constexpr int kCtrClaim = 16;   // [2][8] 64-bit per-XCD claim counters of the GEMM1 and GEMM2 tile kernels
constexpr int kCtrLeft = 48;    // [2] their work-groups that have left
constexpr int kCtrOrder = 64;   // [32] experts by descending item rows: first item | items << 16
constexpr int kNumCounters = 96;
static_assert(kCtrClaim % 2 == 0 && kCtrClaim + 32 <= kCtrLeft && kCtrLeft + 2 <= kCtrOrder &&
              kCtrOrder + kExpertsLocal <= kNumCounters, "control block");

// Rows of a work item of the tile GEMMs: gemm_tile_kernel has an instance for items of up to
// 128 rows and one for items of up to 160 (10 row groups of 16, the largest whose ring fits LDS).
constexpr int kTileItemRowsMid = 128;
constexpr int kTileItemRowsLarge = 160;

// Rows (assignments) per GEMM work item for a call with T tokens. Tile-path items hold up to
// 128 rows below 4096 tokens and up to 160 from there: larger items move fewer bytes per
// flop, but at mid-size batches the fewer, longer units balance worse over the CUs (measured:
// T=1024 GEMM1 170 us with 128-row items against 196 us with 160; T=8192 342 against 319).
// Batches up to kStreamMaxTokens run the wavefront-granular streaming GEMMs (items of 16 or
// 32 rows), larger ones the tile GEMMs.
constexpr int kStreamMaxTokens = 256;
// The tile GEMM2 reads each bucket row's destination (row_dest), which only place_kernel
// writes: every batch of the tile path takes the multi-work-group dispatch.
static_assert(kSinglePassTokens <= kStreamMaxTokens, "tile-path batches are dispatched by place_kernel");

inline int rows_per_item_for(int T) {
  if (T <= 64) return 16;
  if (T <= kStreamMaxTokens) return 32;
  if (T < 4096) return kTileItemRowsMid;
  return kTileItemRowsLarge;
}

// Columns per requantisation scale of the GEMM1 output: the reference's 64 (kernel.py:131-135)
// with items of up to 128 rows (below 4096 tokens), 128 with the 160-row items of larger
// batches (one activation scale, and one MFMA per fragment, per 128-wide K block of the tile
// GEMM2).
inline int requant_block_for(int rows_per_item) { return rows_per_item <= kTileItemRowsMid ? 64 : 128; }

int compute_layout(int32_t T, moe_fp8_layout* out);

// Parameters of the routing/dispatch kernels.
struct RouteParams {
  const float* logits;
  const void* bias;
  int bias_dtype;
  int T;
  int offset;
  float rsf;
  int skip_routing;
  int single_pass;
  int nblocks;
  int rows_per_item;
  int max_items;
  int32_t* topk_ids;
  float* topk_w;
  int32_t* expert_count;
  int32_t* expert_start;
  int32_t* sorted_token;
  float* sorted_weight;
  int32_t* sorted_slot;
  int32_t* token_nlocal;
  int32_t* slot_rank;
  // [N_max] output destination of each bucket row for the tile GEMM2 (place_kernel): the token
  // when it has one local assignment, else -1 - its flat slot
  int32_t* row_dest;
  int32_t* block_count;  // [nblocks, 32] expert histogram of each routing work-group
  int32_t* work_items;   // [max_items, 4]
  int32_t* counters;
};

struct GemmParams {
  const uint8_t* hidden;       // [T, 7168]
  const float* hidden_scale;   // [56, T]
  const uint8_t* w13;          // [32, 4096, 7168]
  const float* w13_scale;      // [32, 32, 56]
  const uint8_t* w2;           // [32, 7168, 2048]
  const float* w2_scale;       // [32, 56, 16]
  int T;
  int max_items;
  const int32_t* work_items;
  int32_t* counters;           // read-only but for the tile kernels' claim counters
  const int32_t* sorted_token;
  const float* sorted_weight;
  const int32_t* sorted_slot;
  const int32_t* token_nlocal;
  // [N_max] output destination of each bucket row on the tile path, as the dispatch wrote it:
  // the token when it has one local assignment (its output row is written directly), else
  // -1 - its flat slot (the row is parked for the combine)
  const int32_t* row_dest;
  uint8_t* act;                // [N_max, 2048]
  float* act_scale;            // [N_max, 2048 / requantisation block]
  float* partial;              // [T*8, 7168]
  float* swiglu;               // [N_max, 2048] (decode path)
  void* out;                   // [T, 7168]
  int out_dtype;
  const int32_t* topk_ids;
  int offset;
};

hipError_t launch_route_dispatch(const RouteParams& p, hipStream_t s);
hipError_t launch_route(const RouteParams& p, hipStream_t s);
// packed (items of up to 32 rows): p.w13 is the packed copy of W13 (moe_fp8_pack_weights).
hipError_t launch_gemm1(const GemmParams& p, int rows_per_item, bool packed, hipStream_t s);
// packed: p.w13 is the packed copy of W13 (moe_fp8_pack_weights).
hipError_t launch_gemm1_dispatch(const GemmParams& p, const RouteParams& rp, bool packed, hipStream_t s);
hipError_t launch_requant(const GemmParams& p, int rows_per_item, hipStream_t s);
// packed (items of up to 32 rows): p.w2 is the packed copy of W2.
hipError_t launch_gemm2(const GemmParams& p, int rows_per_item, bool packed, hipStream_t s);
// The packed copy of W13 and W2 read by the decode kernels (moe_fp8_pack_weights).
size_t packed_weights_bytes();
hipError_t launch_pack_weights(const uint8_t* w13, const uint8_t* w2, uint8_t* packed, hipStream_t s);
hipError_t launch_combine(const GemmParams& p, int rows_per_item, hipStream_t s);
hipError_t launch_gemm1_tile(const GemmParams& p, int rows_per_item, hipStream_t s);
hipError_t launch_quantize_hidden(const void* x, int dtype, int T, uint8_t* q, float* scale, hipStream_t s);
hipError_t launch_gemm2_tile(const GemmParams& p, int rows_per_item, hipStream_t s);
hipError_t launch_clear_control(int32_t* counters, hipStream_t s);

}  // namespace moe
