/*
 * moe_fp8.h - C ABI of the MI355X (gfx950) fused FP8 block-scale MoE layer.
 *
 * The layer is the DeepSeek-V3 routed MoE with the shapes of the MLSys'26
 * FlashInfer MoE track definition moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048:
 * 256 global experts in 8 groups, top-4 groups, top-8 experts, 32 experts local to
 * this device, hidden size 7168, intermediate size 2048, fp8 e4m3fn operands with
 * 128-wide block scales, bf16 output.
 *
 * Every entry point is stream-ordered on the hipStream_t it is given, performs no
 * host<->device synchronisation and allocates no memory: all temporaries live in a
 * caller-owned workspace of moe_fp8_workspace_bytes(T) bytes. Pointers are device
 * pointers to contiguous row-major buffers, aligned for the widest access the kernels make to
 * them (MOE_FP8_EALIGN otherwise): 16 bytes for the logits, hidden states, weights, packed
 * weights, an fp32 output and the quantiser's input; 8 for a bf16 output and the quantiser's
 * fp8 output; 4 for scales and an fp32 bias; 2 for a bf16 or fp16 bias; 256 for the workspace
 * (every allocation of hipMalloc or torch qualifies). Return value: 0 on success, a negative
 * MOE_FP8_E* code otherwise (moe_fp8_strerror() gives the text). Arguments are checked
 * before anything is launched, so on every error but MOE_FP8_ELAUNCH nothing has been
 * launched; MOE_FP8_ELAUNCH reports a launch that HIP rejected, possibly after earlier
 * kernels of the same call were queued (the output is then undefined).
 *
 * Reference interface replaced: run() in kernel.py:562-729 (nikhilnd/mlsys26-flashinfer-moe),
 * and the stages it calls (kernel.py:624-639 routing, 649-661 dispatch and tile schedule,
 * 663-693 token pack + GEMM1, 695-729 GEMM2 + finalize).
 */
#ifndef MOE_FP8_H_
#define MOE_FP8_H_

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layer constants; kernel.py:577-588. */
#define MOE_FP8_HIDDEN          7168
#define MOE_FP8_INTER           2048
#define MOE_FP8_EXPERTS_GLOBAL  256
#define MOE_FP8_EXPERTS_LOCAL   32
#define MOE_FP8_TOP_K           8
#define MOE_FP8_N_GROUP         8
#define MOE_FP8_TOPK_GROUP      4
#define MOE_FP8_BLOCK           128
#define MOE_FP8_H_BLOCKS        (MOE_FP8_HIDDEN / MOE_FP8_BLOCK)       /* 56 */
#define MOE_FP8_I_BLOCKS        (MOE_FP8_INTER / MOE_FP8_BLOCK)        /* 16 */
#define MOE_FP8_G1_BLOCKS       (2 * MOE_FP8_INTER / MOE_FP8_BLOCK)    /* 32 */

/* routing_bias element type; kernel.py:595 accepts float32, bfloat16 and float16. */
#define MOE_FP8_BIAS_F32   0
#define MOE_FP8_BIAS_BF16  1
#define MOE_FP8_BIAS_F16   2

/* hidden_dtype of moe_fp8_quantize_hidden: the element type of the unquantised states. */
#define MOE_FP8_HIDDEN_F32   0
#define MOE_FP8_HIDDEN_BF16  1
#define MOE_FP8_HIDDEN_F16   2

/* output element type. The reference copies its fp32 accumulator into the caller's
 * tensor (kernel.py:729); bf16 is the contract type, fp32 is offered so that an
 * fp32 destination receives the unrounded sums as it would from the reference. */
#define MOE_FP8_OUT_BF16   0
#define MOE_FP8_OUT_F32    1

/* Error codes. */
#define MOE_FP8_OK                  0
#define MOE_FP8_EINVAL_POINTER     -1  /* a required pointer is NULL */
#define MOE_FP8_EINVAL_TOKENS      -2  /* num_tokens < 0 or too large */
#define MOE_FP8_EWORKSPACE         -3  /* workspace NULL or smaller than moe_fp8_workspace_bytes */
#define MOE_FP8_EINVAL_BIAS_DTYPE  -4
#define MOE_FP8_EINVAL_OUT_DTYPE   -5
#define MOE_FP8_ELAUNCH            -6  /* a HIP launch failed (hipGetLastError) */
#define MOE_FP8_EDEVICE            -7  /* current device is not gfx950 */
#define MOE_FP8_EINVAL_HIDDEN_DTYPE -8 /* hidden_dtype of moe_fp8_quantize_hidden unknown */
#define MOE_FP8_ESTATIC_TOKENS     -9  /* num_tokens > MOE_FP8_STATIC_MAX_TOKENS (moe_fp8_run_static) */
#define MOE_FP8_EPACKED           -10  /* packed weights NULL or smaller than moe_fp8_packed_weights_bytes() */
#define MOE_FP8_EALIGN            -11  /* a pointer is not aligned as the kernels read or write it (above) */

/* Largest num_tokens accepted: keeps every flat index (T*8*7168) inside int64 and
 * the per-token slot index inside int32. */
#define MOE_FP8_MAX_TOKENS         (1 << 20)

/* Arguments of one layer call; the tensor contract of kernel.py:563-607. */
typedef struct moe_fp8_args {
  const float*   routing_logits;       /* [T, 256] fp32                                  */
  const void*    routing_bias;         /* [256] fp32 | bf16 | fp16 (routing_bias_dtype)  */
  int32_t        routing_bias_dtype;   /* MOE_FP8_BIAS_*                                 */
  const uint8_t* hidden_states;        /* [T, 7168] fp8 e4m3fn                           */
  const float*   hidden_states_scale;  /* [56, T] fp32, 1x128 block per token            */
  const uint8_t* gemm1_weights;        /* [32, 4096, 7168] fp8 e4m3fn (gate rows 0..2047, up rows 2048..4095) */
  const float*   gemm1_weights_scale;  /* [32, 32, 56] fp32, 128x128 blocks              */
  const uint8_t* gemm2_weights;        /* [32, 7168, 2048] fp8 e4m3fn                    */
  const float*   gemm2_weights_scale;  /* [32, 56, 16] fp32, 128x128 blocks              */
  int32_t        num_tokens;           /* T                                              */
  int32_t        local_expert_offset;  /* experts [offset, offset+32) are local          */
  float          routed_scaling_factor;
  void*          output;               /* [T, 7168] bf16 or fp32 (output_dtype)          */
  int32_t        output_dtype;         /* MOE_FP8_OUT_*                                  */
} moe_fp8_args;

/* Byte offsets of the intermediate arrays inside the workspace. They are part of
 * the ABI so that callers and tests can read (or, before a later stage, write) the
 * intermediates of a call (moe_fp8_layout). N_max = 8*T is the largest possible number of local
 * (token, expert) assignments.
 *   topk_ids      int32 [T, 8]      selected global expert ids, selection order      (kernel.py:629)
 *   topk_weights  fp32  [T, 8]      renormalised, scaled routing weights            (kernel.py:630)
 *   expert_count  int32 [32]        local assignments per local expert              (kernel.py:357)
 *   expert_start  int32 [33]        CSR offsets into the sorted arrays              (kernel.py:358-360)
 *   sorted_token  int32 [N_max]     token of each assignment, grouped by expert,
 *                                   ascending token inside an expert (deterministic) (kernel.py:364)
 *   sorted_weight fp32  [N_max]     routing weight of each assignment               (kernel.py:365)
 *   sorted_slot   int32 [N_max]     flat slot t*8+k of each assignment
 *   token_nlocal  int32 [T]         number of local assignments of each token
 *   slot_rank     int32 [T*8]       internal: the multi-work-group dispatch's stable ranks
 *   work_items    int32 [max_items, 4]  GEMM work list (expert, first row, rows,
 *                                   first item of the expert | its item count << 16) (kernel.py:384-407)
 *   counters      int32 [96]        [0] number of work items, [1] N; the rest internal
 *                                   (the tile kernels' work-list state)
 *   act           fp8   [N_max, 2048]    SwiGLU output requantised to e4m3fn          (kernel.py:669)
 *   act_scale     fp32  [N_max, 32]    its 1 x requant_block scales, row-major per row,
 *                                        2048/requant_block of them              (kernel.py:670)
 *                 requant_block is 64 below 4096 tokens, the reference's 1x64 block (BLOCK_N_1 =
 *                 64, kernel.py:131-135, :643, scales [32, N]). From 4096 tokens on it is 128, a
 *                 deliberate difference: GEMM2 then applies one activation scale per 128-wide K
 *                 block, like every other operand, with one MFMA per fragment instead of two.
 *                 The parity tests bound the output's distance from fp32 math by that of the
 *                 64-column algorithm (per token at most 2x its maximum error + 1/64).
 *   partial       fp32  [T*8, 7168]      weighted GEMM2 rows of tokens with more than one local
 *                                        assignment, indexed by flat slot, above 64 tokens (0
 *                                        bytes up to 64: the combine happens inside GEMM2)
 *                                                                                     (kernel.py:704)
 *   swiglu        fp32  [N_max, 2048]    SwiGLU output before requantisation; only for
 *                                        T <= 256 (0 bytes otherwise)
 *   row_dest      int32 [N_max]     above 256 tokens, written by the dispatch: GEMM2's output
 *                                   destination of each bucket row, the token when it has one
 *                                   local assignment (its output row is written directly),
 *                                   else -1 - its flat slot (the row is parked in `partial`)
 */
typedef struct moe_fp8_layout {
  size_t total_bytes;
  size_t topk_ids;
  size_t topk_weights;
  size_t expert_count;
  size_t expert_start;
  size_t sorted_token;
  size_t sorted_weight;
  size_t sorted_slot;
  size_t token_nlocal;
  size_t slot_rank;
  size_t block_count;
  size_t work_items;
  size_t counters;
  size_t act;
  size_t act_scale;
  size_t partial;
  size_t swiglu;
  size_t row_dest;
  int32_t num_tokens;
  int32_t max_assignments;   /* N_max = 8*T        */
  int32_t max_work_items;
  int32_t route_blocks;      /* routing work-groups */
  int32_t rows_per_item;     /* GEMM rows (assignments) per work item */
  int32_t requant_block;     /* columns per act_scale entry: 64 below 4096 tokens, else 128 */
  int32_t reserved[2];
} moe_fp8_layout;

/* Workspace size for num_tokens tokens (0 if num_tokens is invalid). */
size_t moe_fp8_workspace_bytes(int32_t num_tokens);

/* Fills *layout for num_tokens tokens. Returns MOE_FP8_OK or MOE_FP8_EINVAL_*. */
int moe_fp8_workspace_layout(int32_t num_tokens, moe_fp8_layout* layout);

/* Clears the workspace's control block with a one-work-group kernel (never a memset, so a
 * call captured into a HIP graph records a kernel node). A freshly allocated workspace must
 * be passed through this once before its first use (so that a GEMM stage run before any
 * dispatch finds no work); every dispatch rewrites the control block before the GEMMs read
 * it, so one workspace is reusable by successive calls on one stream without clearing.
 * Calls that overlap in time must use different workspaces. No counterpart in the
 * reference, whose temporaries are freshly zeroed torch tensors (kernel.py:348, 669-670, 704). */
int moe_fp8_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream);

/* The whole layer: routing, dispatch, GEMM1+SwiGLU+requant, GEMM2+weighted combine.
 * Up to 64 tokens the dispatch is rebuilt inside the GEMM1 kernel instead of launched
 * before it; afterwards the workspace holds the same dispatch arrays as after the stage
 * entry points. Replaces run() (kernel.py:562-729). */
int moe_fp8_run(const moe_fp8_args* args, void* workspace, size_t workspace_bytes,
                hipStream_t stream);

/* moe_fp8_run with stage timing: the same launches, with events[0] recorded on `stream` before
 * stage 1 (routing, and the dispatch above 64 tokens), events[1] before stage 2 (GEMM1, one
 * kernel; up to 64 tokens it also rebuilds the dispatch), events[2] before stage 3
 * (requantisation, GEMM2 and the combine) and events[3] after it. The events must have been
 * created by the caller (hipEventCreate) on the stream's device. With a non-NULL `packed` (the
 * packed copy of args' weights, moe_fp8_pack_weights) it times moe_fp8_run_packed instead.
 * Replaces run() (kernel.py:562-729) like moe_fp8_run; the per-stage split mirrors its routing
 * (:624-639), dispatch + GEMM1 (:649-693) and GEMM2 + finalize (:695-729) sections. */
int moe_fp8_run_profiled(const moe_fp8_args* args, const void* packed, size_t packed_bytes, void* workspace,
                         size_t workspace_bytes, hipStream_t stream, hipEvent_t events[4]);

/* A cached re-layout of the expert weights for the decode path, behind the same tensor
 * contract: the caller keeps passing W13/W2 in their kernel.py:604-607 layout and may, once per
 * weight set, build a packed copy that the streaming GEMMs of batches up to 256 tokens read
 * instead.
 * In the copy each wavefront's MFMA operand for a 128-wide K-step is contiguous (32 bytes per
 * lane, 2 KB per 16-row fragment): W13 as blocks [expert][16 SwiGLU columns][K-step] of 4 KB
 * (the gate rows' fragment, then the up rows'), then W2 as blocks [expert][16 hidden
 * rows][K-step] of 2 KB; lane l of a fragment holds bytes [16(l/16), +16) and
 * [64 + 16(l/16), +16) of the block's row l%16. Scales are not copied. An extension
 * of the path with no counterpart in the reference, whose kernels read the weights row-major
 * (kernel.py:91-102, 222-226). */
#define MOE_FP8_PACKED_MAX_TOKENS 256         /* the largest batch that reads the packed copy */
size_t moe_fp8_packed_weights_bytes(void);   /* 1,409,286,144: the size of W13 plus W2 */

/* Writes the packed copy of args->gemm1_weights and args->gemm2_weights (only those two fields
 * are read) into `packed` on `stream`. */
int moe_fp8_pack_weights(const moe_fp8_args* args, void* packed, size_t packed_bytes, hipStream_t stream);

/* moe_fp8_run with the packed copy of args' weights: up to 256 tokens GEMM1 and GEMM2 stream
 * `packed` instead of args->gemm1_weights / gemm2_weights; above 256 tokens `packed` is not
 * read. The output is bit-identical to moe_fp8_run's (the same arithmetic in the same order).
 * Replaces run() (kernel.py:562-729) like moe_fp8_run. */
int moe_fp8_run_packed(const moe_fp8_args* args, const void* packed, size_t packed_bytes, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* moe_fp8_run without a caller workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference, whose temporaries come from torch's allocator
 * (kernel.py:348-370, 629-630, 669-670, 704). The workspace is a device array inside the
 * library of MOE_FP8_STATIC_SCRATCH_BYTES (6 MiB), one per GPU that loads the library, held
 * until the process ends; it holds the workspace of up to MOE_FP8_STATIC_MAX_TOKENS (64)
 * tokens, and larger batches return MOE_FP8_ESTATIC_TOKENS without launching anything.
 * Nothing is allocated or freed by this call (the first call on a device resolves the
 * array's address and clears its control block with a kernel). Every call on one GPU shares
 * that GPU's array: calls that overlap in time on one GPU (on different streams, or from
 * different threads without ordering) race and give wrong results; calls ordered on one
 * stream are safe, each rewriting what it reads. Results are bit-identical to moe_fp8_run. */
#define MOE_FP8_STATIC_MAX_TOKENS    64
#define MOE_FP8_STATIC_SCRATCH_BYTES (6u << 20)
int moe_fp8_run_static(const moe_fp8_args* args, hipStream_t stream);

/* Stage 1: routing and dispatch. Writes topk_ids/topk_weights, the expert histogram,
 * CSR offsets, sorted permutation and the GEMM work list. With skip_routing != 0 the
 * routing itself is skipped and topk_ids/topk_weights already in the workspace are
 * dispatched (routing_logits and routing_bias may then be NULL).
 * Replaces moe_routing_kernel + build_expert_dispatch + build_tile_schedule
 * (kernel.py:624-639, 649-661, 327-407). */
int moe_fp8_route_dispatch(const moe_fp8_args* args, int32_t skip_routing, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

/* Stage 2: GEMM1 over the gathered tokens of each local expert and SwiGLU (silu of the
 * second half times the first half). One kernel. Reads the dispatch arrays; writes the
 * fp8 intermediate act/act_scale (one scale per row per requant_block columns) when
 * layout.rows_per_item > 32, otherwise the fp32 SwiGLU rows `swiglu`, which stage 3
 * requantises first.
 * Replaces the token pack and moe_gemm1_kernel (kernel.py:663-693, 7-151). */
int moe_fp8_gemm1(const moe_fp8_args* args, void* workspace, size_t workspace_bytes,
                  hipStream_t stream);

/* Stage 3: (when layout.rows_per_item <= 32) requantisation of the fp32 SwiGLU rows to
 * act/act_scale, one scale per layout.requant_block columns; GEMM2 of act against the expert's down projection, weighting by the
 * routing weight and the deterministic per-token combine into args->output (up to 64 tokens
 * in one kernel, above that a separate combine pass over the parked rows).
 * Replaces moe_gemm2_kernel and the finalize copy (kernel.py:695-729, 153-250). */
int moe_fp8_gemm2_combine(const moe_fp8_args* args, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);

/* The step before the layer: quantises hidden states [T, 7168] (element type hidden_dtype)
 * to the layer's activation contract, e4m3fn hidden_fp8 [T, 7168] and fp32 hidden_scale
 * [56, T] (token-minor), per token and 128-column block: scale = max(amax / 448, 1e-12),
 * hidden_fp8 = e4m3(x / scale) rounded to nearest even. No workspace. num_tokens == 0 is
 * a no-op. The reference takes these tensors already quantised (kernel.py:600-603); the
 * formula is its own in-path requantisation (kernel.py:131-135) with 128 columns. */
int moe_fp8_quantize_hidden(const void* hidden, int32_t hidden_dtype, int32_t num_tokens,
                            void* hidden_fp8, float* hidden_scale, hipStream_t stream);

/* Text for a return code. */
const char* moe_fp8_strerror(int code);

/* Library version string. */
const char* moe_fp8_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MOE_FP8_H_ */
