// C ABI of libmoe_fp8: argument checks, workspace layout and the launch sequence.
// run() in kernel.py:562-729 is the interface these entry points replace.
#include <string.h>

#include <atomic>
#include <mutex>

#include "moe_internal.h"

namespace moe {

namespace {

constexpr size_t kAlign = 256;
inline size_t align_up(size_t x) { return (x + kAlign - 1) & ~(kAlign - 1); }

int check_device() {
  // per device: 0 unknown, 1 gfx950, -1 another GPU (concurrent first calls store the same)
  static std::atomic<int> arch_ok[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return MOE_FP8_EDEVICE;
  int v = dev < 64 ? arch_ok[dev].load(std::memory_order_relaxed) : 0;
  if (v == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return MOE_FP8_EDEVICE;
    v = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
    if (dev < 64) arch_ok[dev].store(v, std::memory_order_relaxed);   // devices past 64: uncached
  }
  return v == 1 ? MOE_FP8_OK : MOE_FP8_EDEVICE;
}

// Alignment of a pointer to the widest access the kernels make through it (16-byte vector
// loads and DMAs of the logits, hidden rows, weights and packed weights; 16- or 8-byte output
// stores; 4-byte scale loads; the 256-byte aligned workspace layout).
inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }
constexpr uintptr_t kWorkspaceAlign = 256;

bool args_aligned(const moe_fp8_args* a, bool need_routing) {
  if (need_routing &&
      (!aligned(a->routing_logits, 16) || !aligned(a->routing_bias, a->routing_bias_dtype == MOE_FP8_BIAS_F32 ? 4 : 2)))
    return false;
  return aligned(a->hidden_states, 16) && aligned(a->hidden_states_scale, 4) && aligned(a->gemm1_weights, 16) &&
         aligned(a->gemm1_weights_scale, 4) && aligned(a->gemm2_weights, 16) && aligned(a->gemm2_weights_scale, 4) &&
         aligned(a->output, a->output_dtype == MOE_FP8_OUT_F32 ? 16 : 8);
}

int check_args(const moe_fp8_args* a, bool need_routing, void* ws, size_t ws_bytes,
               moe_fp8_layout* L) {
  if (!a) return MOE_FP8_EINVAL_POINTER;
  int rc = compute_layout(a->num_tokens, L);
  if (rc != MOE_FP8_OK) return rc;
  if (a->num_tokens == 0) return MOE_FP8_OK;
  if (need_routing && (!a->routing_logits || !a->routing_bias)) return MOE_FP8_EINVAL_POINTER;
  if (!a->hidden_states || !a->hidden_states_scale || !a->gemm1_weights || !a->gemm1_weights_scale ||
      !a->gemm2_weights || !a->gemm2_weights_scale || !a->output)
    return MOE_FP8_EINVAL_POINTER;
  if (a->routing_bias_dtype < MOE_FP8_BIAS_F32 || a->routing_bias_dtype > MOE_FP8_BIAS_F16)
    return MOE_FP8_EINVAL_BIAS_DTYPE;
  if (a->output_dtype != MOE_FP8_OUT_BF16 && a->output_dtype != MOE_FP8_OUT_F32)
    return MOE_FP8_EINVAL_OUT_DTYPE;
  if (!args_aligned(a, need_routing)) return MOE_FP8_EALIGN;
  if (!ws || ws_bytes < L->total_bytes) return MOE_FP8_EWORKSPACE;
  if (!aligned(ws, kWorkspaceAlign)) return MOE_FP8_EALIGN;
  return check_device();
}

template <typename T>
T* at(void* ws, size_t off) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + off);
}

RouteParams route_params(const moe_fp8_args* a, const moe_fp8_layout& L, void* ws,
                         int skip_routing) {
  RouteParams p;
  p.logits = a->routing_logits;
  p.bias = a->routing_bias;
  p.bias_dtype = a->routing_bias_dtype;
  p.T = a->num_tokens;
  p.offset = a->local_expert_offset;
  p.rsf = a->routed_scaling_factor;
  p.skip_routing = skip_routing;
  p.single_pass = a->num_tokens <= kSinglePassTokens;
  p.nblocks = L.route_blocks;
  p.rows_per_item = L.rows_per_item;
  p.max_items = L.max_work_items;
  p.topk_ids = at<int32_t>(ws, L.topk_ids);
  p.topk_w = at<float>(ws, L.topk_weights);
  p.expert_count = at<int32_t>(ws, L.expert_count);
  p.expert_start = at<int32_t>(ws, L.expert_start);
  p.sorted_token = at<int32_t>(ws, L.sorted_token);
  p.sorted_weight = at<float>(ws, L.sorted_weight);
  p.sorted_slot = at<int32_t>(ws, L.sorted_slot);
  p.token_nlocal = at<int32_t>(ws, L.token_nlocal);
  p.slot_rank = at<int32_t>(ws, L.slot_rank);
  p.row_dest = at<int32_t>(ws, L.row_dest);
  p.block_count = at<int32_t>(ws, L.block_count);
  p.work_items = at<int32_t>(ws, L.work_items);
  p.counters = at<int32_t>(ws, L.counters);
  return p;
}

GemmParams gemm_params(const moe_fp8_args* a, const moe_fp8_layout& L, void* ws) {
  GemmParams p;
  p.hidden = a->hidden_states;
  p.hidden_scale = a->hidden_states_scale;
  p.w13 = a->gemm1_weights;
  p.w13_scale = a->gemm1_weights_scale;
  p.w2 = a->gemm2_weights;
  p.w2_scale = a->gemm2_weights_scale;
  p.T = a->num_tokens;
  p.max_items = L.max_work_items;
  p.work_items = at<int32_t>(ws, L.work_items);
  p.counters = at<int32_t>(ws, L.counters);
  p.sorted_token = at<int32_t>(ws, L.sorted_token);
  p.sorted_weight = at<float>(ws, L.sorted_weight);
  p.sorted_slot = at<int32_t>(ws, L.sorted_slot);
  p.token_nlocal = at<int32_t>(ws, L.token_nlocal);
  p.row_dest = at<int32_t>(ws, L.row_dest);
  p.act = at<uint8_t>(ws, L.act);
  p.act_scale = at<float>(ws, L.act_scale);
  p.partial = at<float>(ws, L.partial);
  p.swiglu = at<float>(ws, L.swiglu);
  p.out = a->output;
  p.out_dtype = a->output_dtype;
  p.topk_ids = at<int32_t>(ws, L.topk_ids);
  p.offset = a->local_expert_offset;
  return p;
}

// Zeroes the control block with ordinary vector stores: a kernel node, never a memset node,
// when a caller captures the call into a graph.
__global__ __launch_bounds__(64) void clear_control_kernel(int32_t* counters) {
  for (int i = threadIdx.x; i < kNumCounters; i += 64) counters[i] = 0;
}

}  // namespace

hipError_t launch_clear_control(int32_t* counters, hipStream_t s) {
  hipLaunchKernelGGL(clear_control_kernel, dim3(1), dim3(64), 0, s, counters);
  return hipGetLastError();
}

int compute_layout(int32_t T, moe_fp8_layout* out) {
  if (!out) return MOE_FP8_EINVAL_POINTER;
  if (T < 0 || T > MOE_FP8_MAX_TOKENS) return MOE_FP8_EINVAL_TOKENS;
  moe_fp8_layout L;
  memset(&L, 0, sizeof(L));
  const size_t t = (size_t)T;
  const size_t nmax = 8 * t;
  const int blocks = (T + kRouteTokensPerBlock - 1) / kRouteTokensPerBlock;
  const int rpi = rows_per_item_for(T);
  const int max_items = kExpertsLocal + (int)((nmax + rpi - 1) / rpi);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes);
    return o;
  };
  L.counters = take(kNumCounters * sizeof(int32_t));  // first: moe_fp8_workspace_init clears it
  L.topk_ids = take(t * kTopK * sizeof(int32_t));
  L.topk_weights = take(t * kTopK * sizeof(float));
  L.expert_count = take(kExpertsLocal * sizeof(int32_t));
  L.expert_start = take((kExpertsLocal + 1) * sizeof(int32_t));
  L.sorted_token = take(nmax * sizeof(int32_t));
  L.sorted_weight = take(nmax * sizeof(float));
  L.sorted_slot = take(nmax * sizeof(int32_t));
  L.token_nlocal = take(t * sizeof(int32_t));
  L.slot_rank = take(t * kTopK * sizeof(int32_t));
  L.block_count = take((size_t)blocks * kExpertsLocal * sizeof(int32_t));
  L.work_items = take((size_t)max_items * 4 * sizeof(int32_t));
  // Items of up to 32 rows keep GEMM1's fp32 SwiGLU rows for requant_kernel; the tile GEMM1
  // requantises in its epilogue. Up to 128-row items the blocks are 64 columns wide, 128 with
  // 160-row items; the scale array is sized for 64 either way, so that the workspace size
  // stays non-decreasing in T. With 16-row items (up to 64 tokens) GEMM2 combines in LDS: no
  // parked rows.
  const int rb = requant_block_for(rpi);
  L.act = take(nmax * kInter);
  L.act_scale = take(nmax * (kInter / 64) * sizeof(float));
  L.partial = take(rpi == 16 ? 0 : t * kTopK * kHidden * sizeof(float));
  L.swiglu = take(rpi <= 32 ? nmax * kInter * sizeof(float) : 0);
  L.row_dest = take(nmax * sizeof(int32_t));
  L.total_bytes = off;
  // The streaming batches' largest workspace (with its fp32 SwiGLU rows) exceeds the first tile
  // batches' own: every tile batch reserves at least that much, so that the size is
  // non-decreasing in T and a workspace sized for T_max serves every T <= T_max.
  if (T > kStreamMaxTokens) {
    moe_fp8_layout S;
    compute_layout(kStreamMaxTokens, &S);
    if (S.total_bytes > L.total_bytes) L.total_bytes = S.total_bytes;
  }
  L.num_tokens = T;
  L.max_assignments = (int32_t)nmax;
  L.max_work_items = max_items;
  L.route_blocks = blocks;
  L.rows_per_item = rpi;
  L.requant_block = rb;
  *out = L;
  return MOE_FP8_OK;
}

namespace {

// The launch sequence of moe_fp8_run; with `events`, events[i] is recorded on the stream
// before stage i+1 (routing [+ dispatch], GEMM1, requantisation + GEMM2 + combine) and
// events[3] after the last launch.
// packed: the packed copy of W13 and W2 (moe_fp8_pack_weights) or null; read only up to 256
// tokens (MOE_FP8_PACKED_MAX_TOKENS), where the streaming kernels read it instead of args'
// weights.
int run_layer(const moe_fp8_args* args, void* workspace, size_t workspace_bytes, hipStream_t stream,
              hipEvent_t* events, const uint8_t* packed = nullptr) {
  moe_fp8_layout L;
  const int rc = check_args(args, true, workspace, workspace_bytes, &L);
  if (rc != MOE_FP8_OK) return rc;
  if (args->num_tokens == 0) return MOE_FP8_OK;
  const RouteParams rp = route_params(args, L, workspace, 0);
  GemmParams gp = gemm_params(args, L, workspace);
  // the streaming GEMMs (items of up to 32 rows) read the packed copy, the tile GEMMs do not
  static_assert(MOE_FP8_PACKED_MAX_TOKENS == kStreamMaxTokens, "the streaming GEMMs' batches");
  const bool use_packed = packed && L.rows_per_item <= 32;
  if (use_packed) {
    gp.w13 = packed;
    gp.w2 = packed + (packed_weights_bytes() - (size_t)kExpertsLocal * kHidden * kInter);
  }
  auto mark = [&](int i) { return !events || hipEventRecord(events[i], stream) == hipSuccess; };
  if (!mark(0)) return MOE_FP8_ELAUNCH;
  if (args->num_tokens <= kFusedDispatchTokens) {
    // routing, then GEMM1 with the dispatch rebuilt in every work-group: one launch less
    if (launch_route(rp, stream) != hipSuccess || !mark(1)) return MOE_FP8_ELAUNCH;
    if (launch_gemm1_dispatch(gp, rp, use_packed, stream) != hipSuccess || !mark(2)) return MOE_FP8_ELAUNCH;
  } else {
    if (launch_route_dispatch(rp, stream) != hipSuccess || !mark(1)) return MOE_FP8_ELAUNCH;
    if (launch_gemm1(gp, L.rows_per_item, use_packed, stream) != hipSuccess || !mark(2)) return MOE_FP8_ELAUNCH;
  }
  if (launch_requant(gp, L.rows_per_item, stream) != hipSuccess) return MOE_FP8_ELAUNCH;
  if (launch_gemm2(gp, L.rows_per_item, use_packed, stream) != hipSuccess) return MOE_FP8_ELAUNCH;
  if (launch_combine(gp, L.rows_per_item, stream) != hipSuccess || !mark(3)) return MOE_FP8_ELAUNCH;
  return MOE_FP8_OK;
}

// The workspace of moe_fp8_run_static: device memory the library holds itself, one copy per
// GPU that loads the library, for callers that cannot allocate. In host code `scratch` names a
// host-side stand-in, not device memory: its device address comes from hipGetSymbolAddress,
// once per device (StaticScratch), and only that address is ever passed to kernels.
__device__ __align__(256) uint8_t scratch[MOE_FP8_STATIC_SCRATCH_BYTES];

struct StaticScratch {
  std::mutex lock;
  void* ptr[64] = {};   // device address of `scratch` on each device; null until set up
};
StaticScratch g_static;

// The current device's scratch address. The first call on a device resolves it (with that
// device current) and clears its control block with a kernel on `stream`; every later call's
// dispatch rewrites the control block before a GEMM reads it.
int static_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return MOE_FP8_EDEVICE;
  std::lock_guard<std::mutex> guard(g_static.lock);
  if (!g_static.ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return MOE_FP8_ELAUNCH;
    if (launch_clear_control(static_cast<int32_t*>(p), stream) != hipSuccess) return MOE_FP8_ELAUNCH;
    g_static.ptr[dev] = p;
  }
  *out = g_static.ptr[dev];
  return MOE_FP8_OK;
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" {

size_t moe_fp8_workspace_bytes(int32_t num_tokens) {
  moe_fp8_layout L;
  if (compute_layout(num_tokens, &L) != MOE_FP8_OK) return 0;
  return L.total_bytes;
}

int moe_fp8_workspace_layout(int32_t num_tokens, moe_fp8_layout* layout) {
  return compute_layout(num_tokens, layout);
}

int moe_fp8_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!workspace || workspace_bytes < kNumCounters * sizeof(int32_t)) return MOE_FP8_EWORKSPACE;
  if (!aligned(workspace, kWorkspaceAlign)) return MOE_FP8_EALIGN;
  return launch_clear_control(static_cast<int32_t*>(workspace), stream) == hipSuccess ? MOE_FP8_OK
                                                                                      : MOE_FP8_ELAUNCH;
}

int moe_fp8_route_dispatch(const moe_fp8_args* args, int32_t skip_routing, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  moe_fp8_layout L;
  const int rc = check_args(args, !skip_routing, workspace, workspace_bytes, &L);
  if (rc != MOE_FP8_OK) return rc;
  if (args->num_tokens == 0) return MOE_FP8_OK;
  const RouteParams p = route_params(args, L, workspace, skip_routing);
  return launch_route_dispatch(p, stream) == hipSuccess ? MOE_FP8_OK : MOE_FP8_ELAUNCH;
}

int moe_fp8_gemm1(const moe_fp8_args* args, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
  moe_fp8_layout L;
  const int rc = check_args(args, false, workspace, workspace_bytes, &L);
  if (rc != MOE_FP8_OK) return rc;
  if (args->num_tokens == 0) return MOE_FP8_OK;
  const GemmParams p = gemm_params(args, L, workspace);
  return launch_gemm1(p, L.rows_per_item, false, stream) == hipSuccess ? MOE_FP8_OK : MOE_FP8_ELAUNCH;
}

int moe_fp8_gemm2_combine(const moe_fp8_args* args, void* workspace, size_t workspace_bytes,
                          hipStream_t stream) {
  moe_fp8_layout L;
  const int rc = check_args(args, false, workspace, workspace_bytes, &L);
  if (rc != MOE_FP8_OK) return rc;
  if (args->num_tokens == 0) return MOE_FP8_OK;
  const GemmParams p = gemm_params(args, L, workspace);
  if (launch_requant(p, L.rows_per_item, stream) != hipSuccess) return MOE_FP8_ELAUNCH;
  if (launch_gemm2(p, L.rows_per_item, false, stream) != hipSuccess) return MOE_FP8_ELAUNCH;
  return launch_combine(p, L.rows_per_item, stream) == hipSuccess ? MOE_FP8_OK : MOE_FP8_ELAUNCH;
}


int moe_fp8_run(const moe_fp8_args* args, void* workspace, size_t workspace_bytes,
                hipStream_t stream) {
  return run_layer(args, workspace, workspace_bytes, stream, nullptr);
}

int moe_fp8_run_profiled(const moe_fp8_args* args, const void* packed, size_t packed_bytes, void* workspace,
                         size_t workspace_bytes, hipStream_t stream, hipEvent_t events[4]) {
  if (!events || !events[0] || !events[1] || !events[2] || !events[3]) return MOE_FP8_EINVAL_POINTER;
  if (packed && packed_bytes < packed_weights_bytes()) return MOE_FP8_EPACKED;
  if (!aligned(packed, 16)) return MOE_FP8_EALIGN;
  return run_layer(args, workspace, workspace_bytes, stream, events, static_cast<const uint8_t*>(packed));
}

size_t moe_fp8_packed_weights_bytes(void) { return packed_weights_bytes(); }

int moe_fp8_pack_weights(const moe_fp8_args* args, void* packed, size_t packed_bytes, hipStream_t stream) {
  if (!args || !args->gemm1_weights || !args->gemm2_weights) return MOE_FP8_EINVAL_POINTER;
  if (!packed || packed_bytes < packed_weights_bytes()) return MOE_FP8_EPACKED;
  if (!aligned(args->gemm1_weights, 16) || !aligned(args->gemm2_weights, 16) || !aligned(packed, 16))
    return MOE_FP8_EALIGN;
  const int rc = check_device();
  if (rc != MOE_FP8_OK) return rc;
  return launch_pack_weights(args->gemm1_weights, args->gemm2_weights, static_cast<uint8_t*>(packed), stream) ==
                 hipSuccess
             ? MOE_FP8_OK
             : MOE_FP8_ELAUNCH;
}

int moe_fp8_run_packed(const moe_fp8_args* args, const void* packed, size_t packed_bytes, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  if (!packed || packed_bytes < packed_weights_bytes()) return MOE_FP8_EPACKED;
  if (!aligned(packed, 16)) return MOE_FP8_EALIGN;
  return run_layer(args, workspace, workspace_bytes, stream, nullptr, static_cast<const uint8_t*>(packed));
}

int moe_fp8_run_static(const moe_fp8_args* args, hipStream_t stream) {
  if (!args) return MOE_FP8_EINVAL_POINTER;
  if (args->num_tokens < 0) return MOE_FP8_EINVAL_TOKENS;
  if (args->num_tokens > MOE_FP8_STATIC_MAX_TOKENS) return MOE_FP8_ESTATIC_TOKENS;
  if (args->num_tokens == 0) return MOE_FP8_OK;
  // every argument check comes before the first call's clear kernel, so that an error other
  // than MOE_FP8_ELAUNCH never leaves a launch behind (the stand-in pointer is only tested
  // against null here; run_layer checks again with the real address)
  moe_fp8_layout L;
  alignas(kWorkspaceAlign) static uint8_t stand_in;
  int rc = check_args(args, true, &stand_in, MOE_FP8_STATIC_SCRATCH_BYTES, &L);
  if (rc != MOE_FP8_OK) return rc;
  void* ws = nullptr;
  rc = static_scratch(stream, &ws);
  if (rc != MOE_FP8_OK) return rc;
  return run_layer(args, ws, MOE_FP8_STATIC_SCRATCH_BYTES, stream, nullptr);
}

int moe_fp8_quantize_hidden(const void* hidden, int32_t hidden_dtype, int32_t num_tokens, void* hidden_fp8,
                            float* hidden_scale, hipStream_t stream) {
  if (num_tokens < 0 || num_tokens > MOE_FP8_MAX_TOKENS) return MOE_FP8_EINVAL_TOKENS;
  if (num_tokens == 0) return MOE_FP8_OK;
  if (!hidden || !hidden_fp8 || !hidden_scale) return MOE_FP8_EINVAL_POINTER;
  if (hidden_dtype < MOE_FP8_HIDDEN_F32 || hidden_dtype > MOE_FP8_HIDDEN_F16) return MOE_FP8_EINVAL_HIDDEN_DTYPE;
  if (!aligned(hidden, 16) || !aligned(hidden_fp8, 8) || !aligned(hidden_scale, 4)) return MOE_FP8_EALIGN;
  const int rc = check_device();
  if (rc != MOE_FP8_OK) return rc;
  return launch_quantize_hidden(hidden, hidden_dtype, num_tokens, static_cast<uint8_t*>(hidden_fp8), hidden_scale,
                                stream) == hipSuccess
             ? MOE_FP8_OK
             : MOE_FP8_ELAUNCH;
}

const char* moe_fp8_strerror(int code) {
  switch (code) {
    case MOE_FP8_OK: return "success";
    case MOE_FP8_EINVAL_POINTER: return "a required pointer argument is NULL";
    case MOE_FP8_EINVAL_TOKENS: return "num_tokens is negative or exceeds MOE_FP8_MAX_TOKENS";
    case MOE_FP8_EWORKSPACE: return "workspace is NULL or smaller than moe_fp8_workspace_bytes(num_tokens)";
    case MOE_FP8_EINVAL_BIAS_DTYPE: return "routing_bias_dtype must be MOE_FP8_BIAS_F32, _BF16 or _F16";
    case MOE_FP8_EINVAL_OUT_DTYPE: return "output_dtype must be MOE_FP8_OUT_BF16 or MOE_FP8_OUT_F32";
    case MOE_FP8_ELAUNCH: return "a HIP kernel launch failed";
    case MOE_FP8_EDEVICE: return "the current HIP device is not a gfx950 (MI355X) GPU";
    case MOE_FP8_EINVAL_HIDDEN_DTYPE: return "hidden_dtype must be MOE_FP8_HIDDEN_F32, _BF16 or _F16";
    case MOE_FP8_EPACKED: return "packed weights are NULL or smaller than moe_fp8_packed_weights_bytes()";
    case MOE_FP8_EALIGN:
      return "a pointer is not aligned as the kernels access it (16 bytes: logits, hidden states, weights, packed "
             "weights, fp32 output, quantiser input; 8: bf16 output, quantiser output; 4: scales, fp32 bias; "
             "2: bf16/fp16 bias; 256: workspace)";
    case MOE_FP8_ESTATIC_TOKENS:
      return "num_tokens exceeds MOE_FP8_STATIC_MAX_TOKENS (64), the largest batch moe_fp8_run_static's "
             "built-in workspace holds; use moe_fp8_run with a caller workspace";
    default: return "unknown error code";
  }
}

const char* moe_fp8_version(void) { return "moe_fp8 0.1.0 gfx950"; }

}  // extern "C"
