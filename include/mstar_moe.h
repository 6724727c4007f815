/* libmstar_moe -- C-ABI of the MI355X (gfx950) fused Mixture-of-Experts path.
 *
 * Conventions for every entry point
 *   - All tensor arguments are device pointers owned by the caller.  No entry
 *     point allocates, frees or synchronises; work is enqueued on `stream`
 *     (a hipStream_t; NULL means the default stream of the current device).
 *   - Return value: 0 on success, otherwise an MSTAR_* status code.  The
 *     message of the calling thread's last failure is returned by
 *     mstar_moe_last_error().  No C++ exception crosses this boundary.
 *   - Dtype codes: MSTAR_DTYPE_*.  Tensors are dense, row-major, contiguous.
 *   - Launches are graph-capturable: no host reads of device data, all grid
 *     sizes follow from the arguments (never from routing results).
 *
 * Reference citations are `file:line` in mstar-project/mstar.
 */
#ifndef MSTAR_MOE_H_
#define MSTAR_MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSTAR_MOE_ABI_VERSION 1

/* status codes */
#define MSTAR_OK 0
#define MSTAR_INVALID_ARGUMENT 1
#define MSTAR_UNSUPPORTED 2
#define MSTAR_LAUNCH_ERROR 3
#define MSTAR_WORKSPACE_TOO_SMALL 4

/* dtype codes */
#define MSTAR_DTYPE_F32 0
#define MSTAR_DTYPE_BF16 1
#define MSTAR_DTYPE_F16 2
#define MSTAR_DTYPE_I32 3
#define MSTAR_DTYPE_I64 4
#define MSTAR_DTYPE_FP8_E4M3FN 5
/* e4m3fn values stored widened to bf16 (exact: e4m3fn is a subset of bf16);
 * the activation format the decode weight-streaming GEMM reads fastest. */
#define MSTAR_DTYPE_FP8_AS_BF16 6

/* quantisation modes of mstar_fused_moe */
#define MSTAR_QUANT_NONE 0     /* w1/w2 in the activation dtype (bf16/fp16)          */
#define MSTAR_QUANT_FP8_W8A8 1 /* e4m3fn weights, 128x128 block scales; activations   */
                               /* quantised per token-group of 128 inside the call    */
#define MSTAR_QUANT_W4A16 2    /* int4 weights (u = q + 8, 8 per int32, element k in  */
                               /* bits 4*(k%8) of word k/8), bf16 scales per 128 of K */

/* Message for the calling thread's most recent failure ("" if none). */
const char* mstar_moe_last_error(void);
int mstar_moe_abi_version(void);

/* Softmax top-k routing from router logits.
 * Replaces TopKRouter.forward from the logits on
 * (mstar/model/components/moe.py:131-139): fp32 softmax, top-k (ties go to
 * the lower expert index), optional renormalisation (norm_topk_prob).
 * logits [num_tokens, num_experts] fp32 or bf16 -> topk_weights
 * [num_tokens, top_k] fp32 and ids as int32 and/or int64 (either may be NULL,
 * not both).  num_experts <= 1024, top_k <= 64. */
int mstar_moe_topk_softmax(const void* logits, int logits_dtype, int64_t num_tokens,
                           int num_experts, int top_k, int renormalize, float* topk_weights,
                           int32_t* topk_ids_i32, int64_t* topk_ids_i64, void* stream);

/* Fused router: TopKRouter.forward (mstar/model/components/moe.py:114-140)
 * from the hidden states on, in one launch: logits = bf16(hidden . gate_weight^T)
 * (bf16 [num_tokens, hidden_size] x bf16 [num_experts, hidden_size], fp32
 * accumulation -- F.linear), fp32 softmax, top-k (ties to the lower expert
 * index), renormalisation if asked.  topk_weights fp32 [num_tokens, top_k];
 * topk_ids int32 and/or int64 (either may be NULL, not both); logits_out
 * (optional, bf16 [num_tokens, num_experts]) receives the logits.
 * act_dtype must be MSTAR_DTYPE_BF16; hidden_size % 32 == 0,
 * num_experts <= 256, top_k <= 64. */
int mstar_moe_router(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                     const void* gate_weight, int num_experts, int top_k, int renormalize,
                     float* topk_weights, int32_t* topk_ids_i32, int64_t* topk_ids_i64,
                     void* logits_out, void* stream);

/* mstar_moe_topk_softmax plus the per-token-group-128 FP8 quantisation of
 * the same tokens' hidden rows, in one launch (one wave per token): hidden
 * [num_tokens, hidden_size] bf16 -> hidden_q [num_tokens, hidden_size]
 * (MSTAR_DTYPE_FP8_AS_BF16: the e4m3fn values widened to bf16) and
 * hidden_scale [num_tokens, hidden_size/128] fp32 (s = max(amax, 1e-10)/448).
 * The routing step of the decode layer (moe.py:131-139) fused with the
 * activation quantisation of the stripped FP8 path (kernels.py:3-7).
 * hidden_size % 512 == 0. */
int mstar_moe_topk_softmax_quant(const void* logits, int logits_dtype, int64_t num_tokens,
                                 int num_experts, int top_k, int renormalize,
                                 float* topk_weights, int32_t* topk_ids_i32,
                                 int64_t* topk_ids_i64, const void* hidden, int64_t hidden_size,
                                 void* hidden_q, float* hidden_scale, void* stream);

/* Token permutation into expert-aligned blocks.
 * Replaces torch.ops._mstar_moe_C.moe_align_block_size
 * (mstar/utils/fused_moe/csrc/moe_align_block_size.cu:207-282) as called by
 * moe_align_block_size (mstar/utils/fused_moe/align.py:55-103).  Same
 * outputs: sorted_token_ids [sorted_len] (padding = numel), expert_ids
 * [expert_ids_len] (blocks past the end = 0), num_tokens_post_pad [1].  The
 * order inside an expert is ascending slot index (the stable order of
 * align.py:146).  Optional extras: expert_offsets [E+1] (padded starts) and
 * expert_counts [E] (unpadded).  Same errors as the reference: padded
 * expert count must be < 1024 (moe_align_block_size.cu:223). */
int mstar_moe_align_block_size(const void* topk_ids, int ids_dtype, int64_t numel,
                               int num_experts, int block_size, int32_t* sorted_token_ids,
                               int64_t sorted_len, int32_t* expert_ids, int64_t expert_ids_len,
                               int32_t* num_tokens_post_pad, int32_t* expert_offsets,
                               int32_t* expert_counts, void* scratch, size_t scratch_bytes,
                               void* stream);

/* Scratch for mstar_moe_align_block_size's grid-wide path (numel > 4096).
 * With scratch NULL the alignment runs in one workgroup (same result,
 * slower for large numel).  The reference allocates its own cumsum buffer
 * inside the op (moe_align_block_size.cu:230); here the caller passes it. */
int mstar_moe_align_scratch_size(int64_t numel, int num_experts, size_t* bytes);

/* Softmax top-k + alignment in one call: mstar_moe_topk_softmax followed by
 * mstar_moe_align_block_size on its ids (one launch when
 * num_tokens*top_k <= 512, else two).  Replaces the router's
 * softmax/topk/renormalise (mstar/model/components/moe.py:131-139) plus
 * moe_align_block_size (mstar/utils/fused_moe/align.py:55-103) as the
 * reference runs them back to back.  topk_ids_i32 and topk_ids_i64 may be
 * NULL (the int32 ids then live in scratch).  scratch: see
 * mstar_moe_route_scratch_size (required above 512 slots). */
int mstar_moe_route(const void* router_logits, int logits_dtype, int64_t num_tokens,
                    int num_experts, int top_k, int renormalize, float* topk_weights,
                    int32_t* topk_ids_i32, int64_t* topk_ids_i64, int block_size,
                    int32_t* sorted_token_ids, int64_t sorted_len, int32_t* expert_ids,
                    int64_t expert_ids_len, int32_t* num_tokens_post_pad, int32_t* expert_offsets,
                    int32_t* expert_counts, void* scratch, size_t scratch_bytes, void* stream);
int mstar_moe_route_scratch_size(int64_t num_tokens, int num_experts, int top_k, size_t* bytes);

/* out[r, :] = dt(dt(act_f32(gate_up[r, :I])) * gate_up[r, I:]).
 * Replaces act_and_mul_triton (mstar/utils/fused_moe/kernels.py:279-298).
 * activation: 0 = silu, 1 = gelu (tanh). */
int mstar_moe_act_and_mul(const void* gate_up, void* out, int dtype, int64_t rows, int64_t inter,
                          int activation, void* stream);

/* output[t, :] = dt(scale * sum_j fp32(input[t, j, :])).
 * Replaces moe_sum_reduce_triton (mstar/utils/fused_moe/kernels.py:359-393). */
int mstar_moe_sum_reduce(const void* input, void* output, int dtype, int64_t tokens,
                         int64_t top_k, int64_t hidden, float routed_scaling_factor,
                         void* stream);

/* Grouped GEMM over expert-aligned blocks, bf16/fp16 (no quantisation):
 * C[slot, :] = dt(A[slot / top_k, :] . B[e(slot)]^T (* topk_weights[slot])).
 * Replaces invoke_fused_moe_kernel / fused_moe_kernel
 * (mstar/utils/fused_moe/kernels.py:141-218, 36-138).  block_size must be
 * the one given to mstar_moe_align_block_size (16, 32, 64 or 128);
 * any N and K (K and N tails are masked, as kernels.py:97-127 masks them).
 * em = sorted_len. */
int mstar_moe_grouped_gemm(const void* A, const void* B, void* C, const void* topk_weights,
                           int topk_w_dtype, const int32_t* sorted_token_ids,
                           const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                           int64_t N, int64_t K, int64_t em, int64_t num_valid_tokens, int top_k,
                           int mul_routed_weight, int block_size, int dtype, void* stream);

/* Grouped GEMM with the quantised variants and the fused activation -- one
 * stage of mstar_fused_moe, exposed for callers that run the stages
 * themselves (e.g. tensor-parallel shards).  Replaces invoke_fused_moe_kernel
 * (mstar/utils/fused_moe/kernels.py:141-218) and the fp8_w8a8 / int4_w4a16
 * branches the reference stripped from it (kernels.py:3-7).
 *   A: [rows, K] bf16/fp16, or e4m3fn with a_scale [rows, K/128] (tiled path);
 *   B: quant NONE [E, N, K] 16-bit; FP8_W8A8 [E, N, K] e4m3fn + b_scale fp32
 *      [E, ceil(N/128), K/128]; W4A16 [E, N, K/8] int32 + b_scale bf16
 *      [E, N, K/128];
 *   activation = -1: C[slot, :N] = dt(acc (* topk_weights[slot]));
 *   activation = 0 (silu) / 1 (gelu): B rows are [gate; up] (N = 2I) and
 *      C[slot, :I] = dt(dt(act(dt(gate))) * dt(up)) (the act_and_mul fused).
 *   path: 0 = auto, 1 = LDS-tiled (needs expert_ids/num_tokens_post_padded
 *   from mstar_moe_align_block_size with this block_size), 2 = weight
 *   streaming (needs expert_offsets/expert_counts; 16-bit A, quantised B;
 *   FP8 activations are quantised per 128-group on the fly).
 * The A row of a slot is slot / top_k.  Quantised B needs K % 128 == 0; quant
 * NONE takes any K. */
int mstar_moe_gemm(const void* A, int a_dtype, const float* a_scale, const void* B, int quant,
                   const void* b_scale, void* C, int c_dtype, const void* topk_weights,
                   int topk_w_dtype, const int32_t* sorted_token_ids, const int32_t* expert_ids,
                   const int32_t* num_tokens_post_padded, const int32_t* expert_offsets,
                   const int32_t* expert_counts, int num_experts, int64_t N, int64_t K,
                   int64_t em, int64_t num_valid_tokens, int top_k, int mul_routed_weight,
                   int activation, int block_size, int path, void* stream);

/* Decode-sized FP8 grouped GEMM driven directly by the router ids: no
 * alignment step.  The fused_moe_kernel of the reference
 * (mstar/utils/fused_moe/kernels.py:36-138, launched by runner.py:118-152)
 * for the fp8_w8a8 branch it stripped (kernels.py:3-7), as a weight stream:
 * each hit expert's weights are read once.
 *   topk_ids [num_slots] int32/int64 (slot s = token s / top_k);
 *   A: a_dtype BF16 [rows, K] (quantised per group of 128 inside), or
 *      FP8_AS_BF16 [rows, K] with a_scale [rows, K/128] (as written by
 *      mstar_moe_topk_softmax_quant); A row of slot s = s / top_k;
 *   B [E, N, K] e4m3fn, b_scale fp32 [E, ceil(N/128), K/128];
 *   activation -1: C[s, :N] = bf16(acc (* topk_weights[s] if mul_routed));
 *   activation 0/1: B rows [gate; up], C[s, :N/2] = act_and_mul.
 * num_slots <= 1024, K % 128 == 0 with K/128 in {1,2,3,4,6,8,12,16}. */
int mstar_moe_stream_gemm(const void* A, int a_dtype, const float* a_scale, const void* B,
                          const float* b_scale, void* C, const void* topk_weights,
                          int topk_w_dtype, const void* topk_ids, int ids_dtype,
                          int64_t num_slots, int num_experts, int64_t N, int64_t K, int top_k,
                          int mul_routed_weight, int activation, void* stream);

/* The routed experts of the FP8 decode layer in ONE launch: the second of
 * mstar_moe_layer's launches at decode sizes.  The gate_up GEMM (+ SiLU /
 * GeLU-and-mul) and the down GEMM (x routed weight) of
 * fused_experts_impl (mstar/utils/fused_moe/runner.py:118-152, the two
 * invoke_fused_moe_kernel calls) as one weight stream; each workgroup's
 * down work starts as soon as the gate_up work of its experts is done.
 *   hq FP8_AS_BF16 [num_tokens, hidden], hs fp32 [num_tokens, hidden/128]
 *     (as written by mstar_moe_topk_softmax_quant);
 *   topk_weights fp32, topk_ids int32 [num_tokens * top_k] (valid ids);
 *   w1 [E, 2*inter, hidden] e4m3fn, w1_scale fp32 [E, 2*inter/128, hidden/128];
 *   w2 [E, hidden, inter] e4m3fn, w2_scale fp32 [E, hidden/128, inter/128];
 *   act: bf16 [num_tokens * top_k, inter] scratch (the SiLU-and-mul rows);
 *   out_rows: bf16 [num_tokens * top_k, hidden], each slot's down row times its
 *     routed weight (mstar_moe_sum_reduce gives the layer output);
 *   sync: int32 [MSTAR_MOE_LAYER_SYNC_WORDS(num_experts)], ZERO when the
 *     launch starts (it is not cleared again; mstar_moe_layer's routing
 *     launch clears its own): per-expert progress counters, an error word
 *     (sync[num_experts], 1 if a wait gave up) and per-workgroup claim words.
 * Workgroups claim the gate_up work a down wait depends on before waiting,
 * so the launch completes whatever share of the CUs it gets; a wait that
 * still exceeds 100 ms sets the error word and writes NaN rows.
 * Shapes: (hidden, inter) = (2048, 768) or (1024, 384), num_tokens * top_k <= 1024 (otherwise
 * MSTAR_UNSUPPORTED). */
int mstar_moe_stream_layer(const void* hq, const float* hs, const void* w1, const float* w1_scale,
                           const void* w2, const float* w2_scale, const float* topk_weights,
                           const int32_t* topk_ids, int64_t num_tokens, int64_t hidden,
                           int num_experts, int64_t inter, int top_k, int activation, void* act,
                           void* out_rows, int32_t* sync, void* stream);

#define MSTAR_MOE_LAYER_SYNC_WORDS(num_experts) ((((num_experts) + 16) / 16) * 16 + 16 * 1024)

/* The same count as MSTAR_MOE_LAYER_SYNC_WORDS, for bindings that cannot
 * read the macro.  No counterpart in the reference. */
int mstar_moe_layer_sync_words(int num_experts, int64_t* words);

/* Number of waits of the one-launch decode layer kernel (mstar_moe_layer at
 * decode sizes, mstar_moe_stream_layer) that gave up on the current device
 * since the library was loaded (synchronous read).  A wait ends by design
 * (see mstar_moe_stream_layer); one that gave up wrote NaN into the rows of
 * the experts it waited for, so that launch's output is detectably invalid.
 * MSTAR_MOE_ONE_LAUNCH=0 in the environment makes mstar_moe_layer use the
 * two-launch form, which has no waits at all.  No counterpart in the
 * reference (a diagnostic of this library's kernel). */
int mstar_moe_layer_wait_failures(int* count);

/* Testing hook for the one-launch decode layer: the mode of the launches
 * enqueued from now on in this process.  0 normal; 1 odd workgroups do not
 * claim their own gate_up work (as if they were not resident yet), so other
 * workgroups must take it over; 2 every down-phase wait gives up at once
 * (the output rows become NaN and the error word is set).  No counterpart in
 * the reference; for tests only. */
int mstar_moe_debug_layer_test_mode(int mode);

/* Workspace bytes mstar_fused_moe needs for these sizes. */
int mstar_fused_moe_workspace_size(int64_t num_tokens, int64_t hidden, int num_experts,
                                   int64_t inter, int top_k, int quant, int act_dtype,
                                   int reduce_results, size_t* bytes);

/* The whole routed-expert computation: align -> gate_up GEMM (+ fused
 * SiLU-and-mul) -> down GEMM (x routed weight) -> top-k sum.
 * Replaces fused_experts (mstar/utils/fused_moe/runner.py:31-159) and its
 * callers' naive fallback dispatch_experts_fused
 * (mstar/model/components/moe.py:143-185).
 *   hidden [num_tokens, hidden_size]; w1 [E, 2*inter, hidden_size] rows
 *   [gate; up]; w2 [E, hidden_size, inter];
 *   quant = MSTAR_QUANT_FP8_W8A8: w1/w2 e4m3fn, w1_scale fp32
 *     [E, 2*inter/128, hidden/128], w2_scale fp32 [E, hidden/128, inter/128];
 *   quant = MSTAR_QUANT_W4A16: w1 int32 [E, 2*inter, hidden/8], w1_scale bf16
 *     [E, 2*inter, hidden/128]; w2 int32 [E, hidden, inter/8], w2_scale bf16
 *     [E, hidden, inter/128];
 *   topk_weights [num_tokens, top_k] fp32/bf16/fp16; topk_ids int32/int64;
 *   out [num_tokens, hidden_size], or [num_tokens, top_k, hidden_size] when
 *   reduce_results == 0 (runner.py:155-156).
 * Quantised paths: hidden_size and inter must be multiples of 128; the
 * bf16/fp16 path takes any sizes. */
int mstar_fused_moe(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                    const void* w1, const void* w2, int num_experts, int64_t inter, int quant,
                    const void* w1_scale, const void* w2_scale, const void* topk_weights,
                    int topk_w_dtype, const void* topk_ids, int ids_dtype, int top_k,
                    int activation, int reduce_results, void* out, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Workspace bytes mstar_moe_layer needs for these sizes. */
int mstar_moe_layer_workspace_size(int64_t num_tokens, int64_t hidden, int num_experts,
                                   int64_t inter, int top_k, int quant, int act_dtype,
                                   size_t* bytes);

/* A routed MoE layer from the router logits: softmax top-k (+ renormalise)
 * -> align -> gate_up GEMM (+ activation) -> down GEMM (x routed weight) ->
 * top-k sum into out [num_tokens, hidden_size].  Replaces the routed half of
 * SparseMoeBlock.forward after the gate projection
 * (mstar/model/components/moe.py:245-261: TopKRouter from its logits on,
 * then _dispatch -> fused_experts).  Same weight formats as
 * mstar_fused_moe.  topk_weights_out [num_tokens, top_k] fp32 and
 * topk_ids_out [num_tokens, top_k] int64 are optional copies of the routing
 * (the reference router returns them). */
int mstar_moe_layer(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                    const void* router_logits, int logits_dtype, int renormalize, const void* w1,
                    const void* w2, int num_experts, int64_t inter, int quant,
                    const void* w1_scale, const void* w2_scale, int top_k, int activation,
                    void* out, float* topk_weights_out, int64_t* topk_ids_out, void* workspace,
                    size_t workspace_bytes, void* stream);

/* The routed layer from the hidden states: the fused router
 * (mstar_moe_router: gate projection x . gate_weight^T in bf16, softmax,
 * top-k, renormalisation) -> align -> gate_up GEMM (+ activation) -> down
 * GEMM (x routed weight) -> top-k sum, as one call.  Replaces the routed half
 * of SparseMoeBlock.forward whole (mstar/model/components/moe.py:245-261,
 * TopKRouter.forward moe.py:130-140 included).  bf16 hidden and gate_weight
 * [num_experts, hidden_size] (num_experts <= 256, hidden_size % 32 == 0);
 * workspace from mstar_moe_layer_workspace_size; logits_out [num_tokens,
 * num_experts] bf16, topk_weights_out and topk_ids_out are optional. */
int mstar_moe_block(const void* hidden, int act_dtype, int64_t num_tokens, int64_t hidden_size,
                    const void* gate_weight, int renormalize, const void* w1, const void* w2,
                    int num_experts, int64_t inter, int quant, const void* w1_scale,
                    const void* w2_scale, int top_k, int activation, void* out,
                    float* topk_weights_out, int64_t* topk_ids_out, void* logits_out,
                    void* workspace, size_t workspace_bytes, void* stream);

/* mstar_moe_layer without a workspace argument: it allocates nothing
 * (no hipMalloc/hipFree, no allocating library call).  No counterpart in
 * the reference; it is for callers that cannot allocate (code under stream
 * capture, serving loops and harnesses that forbid hipMalloc).  The
 * workspace is a fixed device array of MSTAR_MOE_NOALLOC_SCRATCH_BYTES held
 * by the library on each device until the process ends; sizes whose
 * mstar_moe_layer_workspace_size exceeds it return
 * MSTAR_WORKSPACE_TOO_SMALL (16 MiB covers, e.g., 256 tokens of a 2048 /
 * 128 x 768 / top-8 layer in every quant mode).  All calls on one device
 * share that array: calls that overlap in time on one device (two streams
 * or two threads) race.  Arguments and results as mstar_moe_layer. */
#define MSTAR_MOE_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int mstar_moe_layer_noalloc(const void* hidden, int act_dtype, int64_t num_tokens,
                            int64_t hidden_size, const void* router_logits, int logits_dtype,
                            int renormalize, const void* w1, const void* w2, int num_experts,
                            int64_t inter, int quant, const void* w1_scale, const void* w2_scale,
                            int top_k, int activation, void* out, float* topk_weights_out,
                            int64_t* topk_ids_out, void* stream);

/* Activation quantisation, OCP e4m3fn: per token-group of 128
 * (s = max(amax, 1e-10) / 448, scales [rows, cols/128]) or per token
 * (scales [rows]).  No reference counterpart: the reference's FP8 branches
 * were stripped (mstar/utils/fused_moe/kernels.py:3-7); these produce the
 * activation formats of BASELINE configs 2-4. */
int mstar_quant_fp8_per_token_group(const void* x, int dtype, int64_t rows, int64_t cols,
                                    int group_size, uint8_t* q, float* scales, void* stream);
int mstar_quant_fp8_per_token(const void* x, int dtype, int64_t rows, int64_t cols, uint8_t* q,
                              float* scales, void* stream);

/* out[M, N] bf16 = (a[M, K] . w[N, K]^T) * a_scale[m] * w_scale[n], e4m3fn
 * operands, fp32 accumulation.  Replaces the F.linear of the dense layers
 * (mstar/model/components/distributed/linear.py:101, :412;
 * mstar/model/components/linear.py:94) for W8A8 weights.  K % 128 == 0. */
int mstar_fp8_scaled_mm(const uint8_t* a, const float* a_scale, const uint8_t* w,
                        const float* w_scale, void* out, int64_t M, int64_t N, int64_t K,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSTAR_MOE_H_ */
