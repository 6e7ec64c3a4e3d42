/*
 * exq_hip.h -- C ABI of the MI355X (gfx950) ExQ MoE expert-dispatch library
 * (libexq_hip.so).
 *
 * Plain C: raw device pointers, int64 sizes, a HIP stream handle and a
 * caller-provided workspace.  No torch types cross this boundary.  Every
 * entry point is stream-ordered, performs no host<->device synchronisation,
 * allocates no device memory, and returns an exq_status; on failure the
 * thread-local message from exq_last_error() says what was rejected.
 *
 * Layouts (all row-major, contiguous):
 *   hidden            [T, H]            f16 | bf16
 *   topk_ids          [T, k]            i32 | i64   (ids outside [0, E) are dropped)
 *   topk_weights      [T, k]            f32 | f16 | bf16
 *   INT4 w13 packed   [E, 2I, H/2]      u8: low nibble = even k, high = odd k,
 *                                        nibble = q + 8  (moe_int4_kernel.py:8-16)
 *   INT4 w13 scales   [E, 2I, H/g]      f16 (bits passed as uint16_t)
 *   INT4 w2  packed   [E, H, I/2]       u8
 *   INT4 w2  scales   [E, H, I/g]       f16
 *   w13 rows 0..I-1 are the gate projection, rows I..2I-1 the up projection
 *   (exq_dispatch.cu:36-37).
 */
#ifndef EXQ_HIP_H_
#define EXQ_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXQ_ABI_VERSION 1

typedef enum exq_status {
  EXQ_SUCCESS = 0,
  EXQ_ERROR_INVALID_ARGUMENT = 1,
  EXQ_ERROR_UNSUPPORTED = 2,
  EXQ_ERROR_WORKSPACE_TOO_SMALL = 3,
  EXQ_ERROR_HIP = 4
} exq_status;

typedef enum exq_dtype {
  EXQ_DTYPE_F32 = 0,
  EXQ_DTYPE_F16 = 1,
  EXQ_DTYPE_BF16 = 2,
  EXQ_DTYPE_I32 = 3,
  EXQ_DTYPE_I64 = 4,
  EXQ_DTYPE_U8 = 5,
  EXQ_DTYPE_I8 = 6
} exq_dtype;

/* Precision tiers of the compiled quant plan (exq_artifact.py:25-26). */
typedef enum exq_tier { EXQ_TIER_BF16 = 0, EXQ_TIER_INT8 = 1, EXQ_TIER_INT4 = 2 } exq_tier;

/* hipStream_t; NULL means the default stream. */
typedef void* exq_stream;

/* ---- library ------------------------------------------------------------ */

int exq_abi_version(void);
/* Message describing the last non-success status returned on this thread. */
const char* exq_last_error(void);
const char* exq_status_name(int status);

/* ---- routing preparation ------------------------------------------------ */

/*
 * Router: logits [T, E] (f32 | f16 | bf16) -> topk_ids [T, k] (i32 | i64) and
 * topk_weights [T, k] (f32 | f16 | bf16).  Replaces the routing the reference
 * runs before dispatch (exq/codegen/triton_emitter.py:273-277: F.softmax over
 * the router logits, torch.topk, weights divided by their sum), whose output
 * the SGLang hook receives as dispatch_output.topk_output
 * (exq/runtime/sglang_backend.py:88-90).  Softmax in fp32 (exp(l - max)
 * divided by the sum with IEEE division); experts in descending order of that
 * rounded probability, equal probabilities to the lower id (also where the
 * logits differ: the ranking is torch.topk's over the softmax values);
 * renormalize != 0 divides the k weights by their sum.  E <= 1024,
 * 1 <= k <= min(E, 64).
 */
int exq_topk_softmax(const void* logits, int logits_dtype, int64_t n_tokens,
                     int64_t n_experts, int64_t top_k, int renormalize, void* topk_ids,
                     int ids_dtype, void* topk_weights, int weights_dtype, exq_stream stream);

/*
 * Block-padded expert layout.  Replaces sgl_kernel.moe_align_block_size as
 * called at exq/runtime/sglang_backend.py:102-109 (num_experts = E + 1,
 * block_size = 16).  Bucket b = id + 1 (bucket 0 collects id == -1);
 * cumsum[b+1] = cumsum[b] + ceil(count_b / B) * B; sorted_token_ids holds the
 * slots of each bucket in ascending order (deterministic; sgl_kernel's order
 * inside a bucket is arbitrary) and, if pad_sorted_token_ids, `numel` in
 * every padding entry; expert_ids[blk] = b - 1 for the blocks of bucket b and
 * -1 past the end.  Capacities must be at least numel + num_experts*(B-1)
 * and ceil(that / B); cumsum has num_experts + 1 entries.  num_experts <=
 * 4096.  One work-group up to 2048 ids and 1024 buckets; larger calls run
 * over several work-groups with the same results and no scratch memory.
 */
int exq_moe_align_block_size(const void* topk_ids, int ids_dtype, int64_t numel,
                             int64_t num_experts, int64_t block_size,
                             int32_t* sorted_token_ids, int64_t sorted_capacity,
                             int32_t* expert_ids, int64_t expert_ids_capacity,
                             int32_t* num_tokens_post_pad, int32_t* cumsum,
                             int pad_sorted_token_ids, exq_stream stream);

/*
 * Expert boundaries and compacted slot order from a block-padded slot list.
 * Replaces exq_dispatch_cuda.build_ends_from_slots
 * (exq/kernels/cuda_src/exq_dispatch.cu:181-229, bound at :314).
 * expert_ends[0] = 0, expert_ends[e+1] = number of valid slots (< n_active)
 * routed to experts <= e; sort_order[expert_ends[e] + r] = r-th valid slot of
 * expert e in order of appearance (the reference's atomic-cursor order is
 * arbitrary; this one is deterministic).  No pre-zeroing needed.
 * n_experts <= 4096; above 2048 entries or 1024 experts it runs over several
 * work-groups (same results, no scratch memory).
 */
int exq_build_ends_from_slots(const int32_t* sorted_slot_ids, int64_t em,
                              const int32_t* flat_router, int64_t n_active,
                              int64_t n_experts, int32_t* expert_ends,
                              int64_t* sort_order, exq_stream stream);

/*
 * Stable token->expert sort.  Replaces exq_dispatch_cuda.dispatch
 * (exq_dispatch.cu:99-149, bound at :313) and the device half of
 * sort_tokens_by_expert (exq/kernels/moe_grouped_gemm.py:153-163).
 * n_experts < 4096; ids outside [0, n_experts) sort after every valid id, in
 * slot order.  Up to 2048 ids and 1023 experts one work-group; larger calls
 * run over several work-groups (each recounts every id's bucket, so no
 * scratch memory is needed) with the same results.
 */
int exq_dispatch(const void* router_indices, int ids_dtype, int64_t n, int64_t n_experts,
                 int64_t* sort_order, int64_t* sorted_expert_ids, int32_t* expert_ends,
                 exq_stream stream);

/* ---- row movement and elementwise ---------------------------------------- */

/*
 * out[i, :] = hidden[sort_order[i] / top_k, :].  Replaces
 * exq_dispatch_cuda.gather_hidden (exq_dispatch.cu:234-260, bound at :316).
 * dtype: f32 | f16 | bf16.
 */
int exq_gather_hidden(const void* hidden, int dtype, int64_t n_tokens, int64_t hidden_size,
                      const int64_t* sort_order, int64_t n_active, int64_t top_k,
                      void* out, exq_stream stream);

/*
 * result[t, :] = sum_j w[t, j] * down_out[pos(t*k + j), :] where pos is the
 * inverse of sort_order; fp32 accumulation in the fixed order j = 0..k-1
 * (deterministic; the reference uses fp32 atomics).  Replaces
 * exq_dispatch_cuda.combine (exq_dispatch.cu:262-310, bound at :317).
 * Needs exq_combine_workspace_size(n_active) bytes of workspace.
 */
size_t exq_combine_workspace_size(int64_t n_active);
int exq_combine(const void* down_out, int dtype, const int64_t* sort_order, int64_t n_active,
                const void* router_weights, int weights_dtype, int64_t n_tokens,
                int64_t top_k, int64_t hidden_size, void* result,
                void* workspace, size_t workspace_bytes, exq_stream stream);

/*
 * out[m, j] = silu(x[m, j]) * x[m, I + j] computed in fp32.  Replaces
 * sgl_kernel.silu_and_mul (call sites sglang_backend.py:137-140,
 * moe_int4_kernel.py:398-400).  dtype: f32 | f16 | bf16.
 */
int exq_silu_and_mul(const void* input, int dtype, int64_t rows, int64_t inter,
                     void* out, exq_stream stream);

/* ---- grouped GEMMs over expert-sorted rows ------------------------------ */

/*
 * C[r, :] = A[r, :] @ dequant(W[e])^T for the rows r of each expert segment
 * [expert_ends[e], expert_ends[e+1]).  INT4 weights are dequantised in
 * registers (exact (q-8) values, fp32 group accumulation, fp16 group scale
 * applied in fp32).  Replaces the _moe_gemm_int4_kernel launch of
 * moe_int4_forward (exq/kernels/moe_int4_kernel.py:124-240, 303-326).
 * A and C: f16 | bf16 (same dtype).  K % 32 == 0 and a group size that is a
 * multiple of 32 dividing K (the reference's minimum group is 32,
 * moe_int4_kernel.py:286-290); any N >= 1 (the reference masks the N tail).
 * K, group_size multiples of 128 with N % 32 == 0 take the tiled / grouped
 * kernels, other shapes the general kernel.  exq_moe_gemm_workspace_size
 * covers the token-group list and, for INT4 weights with N % 128 == 0 (the
 * tiled kernel), the per-row group sums of A (n_rows * K / 128 floats).
 */
size_t exq_moe_gemm_workspace_size(int64_t n_rows, int64_t n_experts, int64_t K);
int exq_moe_int4_gemm(const void* a_sorted, int act_dtype, int64_t n_rows, int64_t K,
                      const uint8_t* packed, const uint16_t* scales, int64_t n_experts,
                      int64_t N, int64_t group_size, const int32_t* expert_ends,
                      void* c, void* workspace, size_t workspace_bytes, exq_stream stream);

/*
 * Unquantised grouped GEMM (the BF16-expert semantics).  W [E, N, K] in the
 * activation dtype; expert_mask (nullable) skips experts whose entry is 0.
 * Replaces _moe_gemm_kernel / moe_grouped_gemm
 * (exq/kernels/moe_grouped_gemm.py:47-132, 173-227).
 */
int exq_moe_grouped_gemm(const void* a_sorted, int act_dtype, int64_t n_rows, int64_t K,
                         const void* weights, int64_t n_experts, int64_t N,
                         const int32_t* expert_ends, const int32_t* expert_mask,
                         void* c, void* workspace, size_t workspace_bytes, exq_stream stream);

/* ---- weight quantisation -------------------------------------------------- */

/*
 * INT4 RTN packing of [rows, K] weights (f32 | f16 | bf16), bit-exact with
 * pack_int4_weights / pack_experts_int4 (exq/kernels/moe_int4_kernel.py:37-119):
 * per (row, group) scale = max|w| / 7 in fp32 (IEEE division) floored at fp32
 * eps, q = round-half-even(w / scale) clamped to [-8, 7], nibble q + 8 (even k
 * low), scales stored fp16.  K < group_size collapses to one group of K.
 * Replaces the one-time packing of _get_or_pack (sglang_backend.py:32-60).
 */
int exq_pack_int4(const void* weights, int dtype, int64_t rows, int64_t K,
                  int64_t group_size, uint8_t* packed, uint16_t* scales, exq_stream stream);

/*
 * INT8 per-output-row RTN (exq/eval/quant_shim.py:84-96 rule): scale =
 * max|w| / 127 (fp32, floored at eps), q = round-half-even(w / scale) clamped
 * to [-128, 127]; the scale is stored fp16.
 */
int exq_quantize_int8(const void* weights, int dtype, int64_t rows, int64_t K, int8_t* q,
                      uint16_t* scales, exq_stream stream);

/*
 * Fake quantisation of [rows, K] weights (f32 | f16 | bf16) into `out` (same
 * shape and dtype; may alias `weights`): quantise then dequantise, the
 * accuracy-simulation path of quantize_tensor_int4 / quantize_tensor_int8
 * (exq/eval/quant_shim.py:84-125).  bits = 4: per group of group_size along
 * the row (the reference uses 128 and pads a short last group with zeros,
 * which leaves its max|w| unchanged), scale = max|w| / 7; bits = 8: per row,
 * scale = max|w| / 127.  Scales in fp32 (IEEE division) floored at fp32 eps,
 * q = round-half-even(w / scale) clamped to [-8, 7] / [-128, 127], out =
 * q * scale rounded once to the dtype.
 */
int exq_fake_quant(const void* weights, int dtype, int64_t rows, int64_t K, int bits,
                   int64_t group_size, void* out, exq_stream stream);

/* ---- fused MoE layer ----------------------------------------------------- */

typedef struct exq_moe_problem {
  int64_t n_tokens;      /* T */
  int64_t hidden_size;   /* H */
  int64_t inter_size;    /* I (per expert) */
  int64_t n_experts;     /* E routed experts */
  int64_t top_k;         /* k */
  int64_t n_shared;      /* always-on experts, ids E..E+n_shared-1, weight 1 */
  int64_t group_size;    /* INT4 group size: a multiple of 32 dividing H and I */
  int act_dtype;         /* hidden / out: f16 | bf16 */
  int ids_dtype;         /* i32 | i64 */
  int weights_dtype;     /* f32 | f16 | bf16 */
} exq_moe_problem;

/*
 * Weight banks of a mixed-precision layer.  tier[e] / index[e] (device
 * arrays of n_experts + n_shared entries) select the bank and the row in it:
 * tier[e] must be 0, 1 or 2 and index[e] a row of that tier's bank, in
 * [0, 2^30).  The arrays live on the device, so the library does not check
 * them; other values make the layer read outside the banks (the Python
 * MixedExpertBank checks them when it is built).
 * BF16 bank: weights in the activation dtype.  INT8 bank: int8 weights with
 * one fp16 scale per output row (quant_shim.py:84-96 semantics).  INT4 bank:
 * the packed layout above.
 */
typedef struct exq_expert_bank {
  const int8_t* tier;
  const int32_t* index;
  const void* bf16_w13;             /* [nb, 2I, H] */
  const void* bf16_w2;              /* [nb, H, I]  */
  const int8_t* int8_w13;           /* [n8, 2I, H] */
  const uint16_t* int8_w13_scales;  /* [n8, 2I]    */
  const int8_t* int8_w2;            /* [n8, H, I]  */
  const uint16_t* int8_w2_scales;   /* [n8, H]     */
  const uint8_t* int4_w13;          /* [n4, 2I, H/2]   */
  const uint16_t* int4_w13_scales;  /* [n4, 2I, H/g]   */
  const uint8_t* int4_w2;           /* [n4, H, I/2]    */
  const uint16_t* int4_w2_scales;   /* [n4, H, I/g]    */
} exq_expert_bank;

/*
 * Workspace bytes needed by the fused entry points for this problem.  The
 * first bytes of a fused-layer workspace hold the combine counters of the
 * decode kernels (T <= 64); each call's first kernel clears them, so the
 * workspace needs no zero fill (any contents will do), but a workspace must
 * not be shared by calls that may run concurrently.
 */
size_t exq_moe_workspace_size(const exq_moe_problem* problem);

/*
 * The whole INT4 MoE layer: routing preparation, gate/up INT4 GEMM fused with
 * SiLU-and-mul, down INT4 GEMM, top-k weighted combine.  Decode batches
 * (T <= 64) run as two kernels (gate/up + SiLU, down + combine) that route
 * for themselves (for one or two tokens the down kernel owns output rows
 * across all routed slots and sums them itself; from 32 tokens, or when large
 * experts split each down contraction four or more ways, a third launch
 * combines); larger batches as routing plan + two grouped MFMA GEMMs +
 * combine.  H, I multiples of 32 and a group size that is a multiple of 32
 * dividing both; shapes whose H, I or group size is not a multiple of 128
 * run as routing plan + the general kernels + combine at every batch size
 * (the mixed-precision layer keeps the 128-multiples).  Replaces the
 * pipeline of _exq_forward_cuda (exq/runtime/sglang_backend.py:65-158:
 * moe_align_block_size -> build_ends_from_slots -> gather_hidden -> GEMM1 ->
 * silu_and_mul -> GEMM2 -> combine) and moe_int4_full_forward
 * (exq/kernels/moe_int4_kernel.py:330-426).  No host synchronisation.
 * Numerics: INT4 products are exact (q-8) * x sums over each scale group,
 * scaled in fp32, except in batches above 64 tokens whose experts average 512
 * or more routed rows: there each weight is dequantised to the activation
 * dtype, (q-8) * s rounded once (the value the reference's kernel multiplies
 * in fp16, moe_int4_kernel.py:211-233), which adds about 0.3 % relative error
 * with bf16 activations.
 * sort_order_out [T*k] (i64) and expert_ends_out [E+1] (i32) are optional
 * copies of the routing preparation over the routed experts: sort_order_out
 * lists routed slots t*k + j (shared experts are not in it), the entries past
 * expert_ends_out[E] are left unwritten (slots whose id is outside [0, E)).
 */
int exq_moe_int4_fused_forward(const exq_moe_problem* problem, const void* hidden,
                               const void* topk_ids, const void* topk_weights,
                               const uint8_t* w13_packed, const uint16_t* w13_scales,
                               const uint8_t* w2_packed, const uint16_t* w2_scales,
                               void* out, int64_t* sort_order_out, int32_t* expert_ends_out,
                               void* workspace, size_t workspace_bytes, exq_stream stream);

/*
 * Mixed-precision layer: BF16, INT8 and INT4 experts of one layer dispatched
 * by the compiled quant plan in one launch sequence (the reference packs
 * every expert INT4 and ignores the plan, sglang_backend.py:38-45; the plan
 * reader is exq/kernels/exq_artifact.py:96-192).  Shared experts
 * (n_shared > 0) are applied to every token with weight 1.
 */
int exq_moe_mixed_forward(const exq_moe_problem* problem, const void* hidden,
                          const void* topk_ids, const void* topk_weights,
                          const exq_expert_bank* bank, void* out,
                          int64_t* sort_order_out, int32_t* expert_ends_out,
                          void* workspace, size_t workspace_bytes, exq_stream stream);

/*
 * The INT4 layer of exq_moe_int4_fused_forward without a workspace argument:
 * no counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Its scratch is a device array of
 * EXQ_NOALLOC_SCRATCH_BYTES held by every GPU the library runs on until the
 * process ends; a problem whose exq_moe_workspace_size exceeds it is rejected
 * with EXQ_ERROR_WORKSPACE_TOO_SMALL before any launch.  The call allocates
 * nothing (no hipMalloc / hipFree).  Every call on one GPU shares that GPU's
 * scratch, so calls that may overlap on one GPU (other streams, other
 * threads) race: serialise them.  Nothing in the scratch needs to start at
 * zero (the layer's first kernel clears its counters).  The first call on a
 * device looks the scratch up and must be made outside graph capture (under
 * capture it returns EXQ_ERROR_UNSUPPORTED and launches nothing); a call with
 * n_tokens = 0 is enough, and later calls may be captured and replayed.  Same
 * arguments and results otherwise.
 */
#define EXQ_NOALLOC_SCRATCH_BYTES (64u << 20)
int exq_moe_int4_fused_forward_noalloc(const exq_moe_problem* problem, const void* hidden,
                                       const void* topk_ids, const void* topk_weights,
                                       const uint8_t* w13_packed, const uint16_t* w13_scales,
                                       const uint8_t* w2_packed, const uint16_t* w2_scales,
                                       void* out, int64_t* sort_order_out,
                                       int32_t* expert_ends_out, exq_stream stream);

/*
 * Measurement hook (no counterpart in the reference, whose harness times whole
 * calls with perf_counter, exq/eval/bench.py:15-46).  When set on the calling
 * thread, the next fused / mixed forward records hipEvent_t events on the
 * call's stream.  Decode batches (two kernels): events[0] / events[1] are the
 * start / stop of the gate/up kernel and events[2] / events[3] those of the
 * down kernel, recorded by the launches themselves (hipExtLaunchKernelGGL),
 * so each pair times exactly one kernel.  Larger batches: events[0] before the
 * routing kernel, events[1] before the gate/up kernel, events[2] before the
 * down kernel and events[3] after the combine kernel.  Pass (NULL, 0) to
 * disable.  The hook is consumed by one call.
 */
int exq_set_stage_events(void* const* events, int n_events);

/*
 * Measurement hook (no counterpart in the reference): the streaming-read
 * ceiling.  Reads `bytes` (a multiple of 16) from `buf` with 16-byte
 * nontemporal loads (faster from HBM than the default cache policy),
 * grid-strided over min(sink_words, 8192) work-groups of 256 threads, and
 * XORs each work-group's fold into sink[work-group] (so nothing is dead);
 * bench.py times it on a buffer far larger than the Infinity Cache to report
 * the HBM read rate the decode kernels are measured against.
 */
int exq_stream_read(const void* buf, int64_t bytes, uint32_t* sink, int64_t sink_words,
                    exq_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* EXQ_HIP_H_ */
