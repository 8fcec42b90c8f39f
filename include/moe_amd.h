/*
 * moe_amd — C ABI of the MI355X (gfx950) MoE expert-layer kernels.
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t passed
 * as `void*` (the caller's current stream), enqueues its kernels on that
 * stream and returns an int status (MOE_OK or a negative MOE_ERR_*).  Nothing
 * synchronises the device and nothing reads device data back to the host.
 * The library allocates no device memory: scratch comes from the caller
 * through `workspace` arguments sized by the *_workspace_size() queries.
 * moe_amd_last_error() returns the text of the last failure on this thread.
 *
 * Shapes: T tokens, H hidden, E experts, K top-k, I intermediate (moe
 * intermediate size), S = T*K routed rows.  Layouts are row-major:
 *   hidden_states [T,H], gate_up_proj [E,2I,H] (rows 0..I-1 gate, I..2I-1 up),
 *   down_proj [E,H,I], topk_index [T,K] int64, topk_weights [T,K].
 * Routed rows are ordered by expert (stable: token-major inside an expert);
 * offsets[e] is the first routed row of expert e, offsets[E] the number of
 * rows that belong to real experts (ids outside [0,E) are "sentinels": they
 * sort behind every expert and contribute zero, as expert-parallel sentinels
 * do in transformers' grouped_mm backend).
 *
 * Reference interfaces (leonmodal/moe at its pinned transformers 5.x):
 *   router      src/models/modeling_qwen3_moe.py:266-275 (Qwen3MoeTopKRouter)
 *               src/models/router.py:103-155           (DeepSeekRouter)
 *   experts     transformers/integrations/moe.py:377-478 (grouped_mm_experts_forward)
 *               registered through ExpertsInterface (integrations/moe.py:481-506)
 */
#ifndef MOE_AMD_H
#define MOE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MOE_OK = 0,
  MOE_ERR_ARG = -1,         /* bad shape or argument            */
  MOE_ERR_DTYPE = -2,       /* unsupported dtype code           */
  MOE_ERR_ALIGN = -3,       /* pointer not 16-byte aligned      */
  MOE_ERR_WORKSPACE = -4,   /* workspace missing or too small   */
  MOE_ERR_HIP = -5,         /* HIP runtime / launch error       */
  MOE_ERR_UNSUPPORTED = -6  /* valid request this build lacks   */
};

enum { MOE_DTYPE_F32 = 0, MOE_DTYPE_BF16 = 1 };

/* Row-tile heights for which moe_amd_permute() writes tile prefix sums. */
enum { MOE_NUM_TILE_SIZES = 3 };

int moe_amd_abi_version(void);
const char* moe_amd_last_error(void);

/* ---------------------------------------------------------------- router */

/* The gating linear: logits[T,E] = hidden_states[T,H] . weight[E,H]^T with
 * bf16 inputs and fp32 accumulation (MFMA).  logits_dtype BF16 rounds the
 * result to bf16, as F.linear on bf16 tensors does for the softmax router
 * (Qwen3MoeTopKRouter.forward, src/models/modeling_qwen3_moe.py:268-270);
 * F32 keeps the fp32 sums, which is F.linear(h.float(), W.float()) of the
 * DeepSeek router (src/models/router.py:107-109) -- a bf16 x bf16 product is
 * exact in fp32, so only the summation order differs.  H multiple of 64,
 * E multiple of 8. */
int moe_amd_router_linear(const void* hidden_states, const void* weight, int64_t T, int E, int H,
                          void* logits, int logits_dtype, void* stream);

/* The gating linear with the softmax router fused into its epilogue:
 * probs[T,E] fp32, topk_weights[T,K] fp32 and topk_index[T,K] int64 exactly
 * as moe_amd_router_linear (bf16 logits) followed by
 * moe_amd_router_softmax_topk (same logits, same top-K arithmetic, bit for
 * bit), without the logits' round trip through memory; the bf16 logits are
 * also written when `logits` is not NULL.  Replaces F.linear + softmax +
 * topk + renormalisation of Qwen3MoeTopKRouter.forward
 * (src/models/modeling_qwen3_moe.py:268-274); logit_offset [E] (may be
 * NULL) is added before the softmax.  Shapes: H multiple of 64, E of 8,
 * and 64 < E <= 128 with K <= 8 or 128 < E <= 256 with K <= 16 (else
 * MOE_ERR_UNSUPPORTED). */
int moe_amd_router_linear_softmax_topk(const void* hidden_states, const void* weight, int64_t T,
                                       int E, int H, const float* logit_offset, int K,
                                       int renormalize, float* probs, float* topk_weights,
                                       int64_t* topk_index, void* logits, void* stream);

/* The gating linear with the DeepSeek-V3 router fused into its epilogue:
 * scores[T,E] fp32, topk_weights[T,K] (weights_dtype) and topk_index[T,K]
 * int64 exactly as moe_amd_router_linear (fp32 logits) followed by
 * moe_amd_router_sigmoid_topk with the same arguments (same logits, same
 * selection and weight arithmetic, bit for bit), without the fp32 logits'
 * round trip through memory; the fp32 logits are also written when `logits`
 * is not NULL, and tokens_per_expert (may be NULL) accumulates the
 * selection counts.  Replaces F.linear(h.float(), W.float()), sigmoid,
 * biased (group-limited) top-K, renormalisation and scaling of
 * DeepSeekRouter.forward (src/models/router.py:107-152; group_limited_topk
 * :22-70).  Shapes: H multiple of 64, E multiple of 8 with E <= 128, K <= 8,
 * num_groups 0 (flat) or at most 8 (else MOE_ERR_UNSUPPORTED). */
int moe_amd_router_linear_sigmoid_topk(const void* hidden_states, const void* weight, int64_t T,
                                       int E, int H, const float* expert_bias, int K,
                                       int renormalize, float scaling_factor, int num_groups,
                                       int group_topk, float* scores, void* topk_weights,
                                       int weights_dtype, int64_t* topk_index,
                                       float* tokens_per_expert, float* logits, void* stream);

/* The gating linear's input gradient for bf16 logits: d_x[T,H] =
 * bf16(d_logits[T,E] . weight[E,H]) (bf16 inputs, fp32 accumulation) -- the
 * grad_input of F.linear's backward (autograd of
 * src/models/modeling_qwen3_moe.py:268-270).  H multiple of 256, E of 8. */
int moe_amd_router_linear_backward_dx(const void* d_logits, const void* weight, int64_t T, int E,
                                      int H, void* d_x, void* stream);

/* The gating linear's weight gradient for bf16 logits: d_weight[E,H] =
 * bf16(sum_t d_logits[t,:]^T hidden_states[t,:]), the grad_weight of
 * F.linear's backward.  Split over token chunks (one fp32 partial per chunk
 * in the caller's workspace, moe_amd_router_linear_backward_dw_workspace_size
 * bytes), reduced in chunk order: deterministic.  H multiple of 256; E a
 * multiple of 8. */
size_t moe_amd_router_linear_backward_dw_workspace_size(int64_t T, int E, int H);
int moe_amd_router_linear_backward_dw(const void* d_logits, const void* hidden_states, int64_t T,
                                      int E, int H, void* workspace, size_t workspace_bytes,
                                      void* d_weight, void* stream);

/* Both gradients of the gating linear for fp32 logits: the DeepSeek router's
 * F.linear(h.float(), W.float()) (src/models/router.py:107-109), whose
 * autograd computes d_x = bf16(d_logits . W) and d_weight =
 * bf16(d_logits^T . h) in fp32 arithmetic (replaces those two fp32 GEMMs).
 * Each fp32 d_logits element g is split into two bf16 terms, hi = bf16(g)
 * and lo = bf16(g - hi), |g - hi - lo| <= 2^-18 |g|; both gradients then run
 * on the bf16 MFMA kernels (exact products, fp32 sums) with the two terms
 * stacked along the reduction: d_x = [hi|lo] . [W;W], d_weight = the hi and
 * lo partial products added in fp32 before the one bf16 rounding.  d_x or
 * d_weight may be NULL (that gradient is skipped).  d_logits [T,E] fp32;
 * hidden_states [T,H], weight [E,H], d_x, d_weight bf16.  H multiple of 256,
 * E of 32.  Workspace: moe_amd_router_linear_backward_f32_workspace_size
 * bytes. */
size_t moe_amd_router_linear_backward_f32_workspace_size(int64_t T, int E, int H);
int moe_amd_router_linear_backward_f32(const float* d_logits, const void* hidden_states,
                                       const void* weight, int64_t T, int E, int H,
                                       void* workspace, size_t workspace_bytes, void* d_x,
                                       void* d_weight, void* stream);

/* Softmax router after the gating linear: probs = softmax(float(logits) +
 * logit_offset) over E, top-K (value descending, lower expert id first on
 * equal values), optional renormalisation by the top-K sum (no epsilon).
 * Replaces Qwen3MoeTopKRouter.forward lines 269-274 of
 * src/models/modeling_qwen3_moe.py.  logit_offset [E] may be NULL.
 * tokens_per_expert [E] (fp32, may be NULL) is incremented by the selection
 * counts.  Outputs: probs [T,E] fp32, topk_weights [T,K] fp32,
 * topk_index [T,K] int64. */
int moe_amd_router_softmax_topk(const void* logits, int logits_dtype, const float* logit_offset,
                                int64_t T, int E, int K, int renormalize, float* probs,
                                float* topk_weights, int64_t* topk_index,
                                float* tokens_per_expert, void* stream);

/* Backward of the above (autograd of softmax -> gather -> renorm).  d_probs
 * (gradient arriving on the returned router_logits, [T,E] fp32) may be NULL.
 * Writes d_logits [T,E] in d_logits_dtype (the logits' dtype). */
int moe_amd_router_softmax_topk_backward(const float* probs, const int64_t* topk_index,
                                         const float* d_topk_weights, const float* d_probs,
                                         int64_t T, int E, int K, int renormalize,
                                         void* d_logits, int d_logits_dtype, void* stream);

/* DeepSeek-V3 router after the fp32 gating linear: scores = sigmoid(logits);
 * selection = top-K of scores + expert_bias (flat, or group-limited when
 * num_groups > 0: groups scored by the sum of their top K/group_topk,
 * group_topk groups kept); weights = gathered unbiased scores, divided by
 * (sum + 1e-20) when renormalize, times scaling_factor when > 0, stored in
 * weights_dtype.  Replaces DeepSeekRouter.forward lines 111-152 of
 * src/models/router.py (group_limited_topk: lines 22-70).
 * tokens_per_expert (may be NULL) accumulates the bincount of line 145. */
int moe_amd_router_sigmoid_topk(const float* logits, const float* expert_bias, int64_t T, int E,
                                int K, int renormalize, float scaling_factor, int num_groups,
                                int group_topk, float* scores, void* topk_weights,
                                int weights_dtype, int64_t* topk_index,
                                float* tokens_per_expert, void* stream);

/* The same router from given scores [T,E] (fp32 values) instead of logits:
 * the reference's path under bf16 autocast, where F.linear(h.float(),
 * W.float()) still yields bf16 logits and torch.sigmoid bf16 scores
 * (src/models/router.py:107-112); the caller passes those scores.  Selection
 * on scores + expert_bias in fp32 (line 116); the weights follow torch's
 * bf16 arithmetic of lines 130-138: the sum of the gathered scores rounded to
 * bf16, + 1e-20 rounded, the quotient and the scaled weight each rounded to
 * bf16.  Nothing is written back to scores. */
int moe_amd_router_sigmoid_topk_scores(const float* scores, const float* expert_bias, int64_t T,
                                       int E, int K, int renormalize, float scaling_factor,
                                       int num_groups, int group_topk, void* topk_weights,
                                       int weights_dtype, int64_t* topk_index,
                                       float* tokens_per_expert, void* stream);

/* Backward of the DeepSeek router's sigmoid -> gather -> renorm -> scale.
 * d_topk_weights is in weights_dtype; d_scores [T,E] fp32 may be NULL.
 * Writes d_logits [T,E] fp32. */
int moe_amd_router_sigmoid_topk_backward(const float* scores, const int64_t* topk_index,
                                         const void* d_topk_weights, int weights_dtype,
                                         const float* d_scores, int64_t T, int E, int K,
                                         int renormalize, float scaling_factor,
                                         float* d_logits, void* stream);

/* ----------------------------------------------------------- permutation */

/* Workspace bytes moe_amd_permute() needs for S routed rows, E experts. */
size_t moe_amd_permute_workspace_size(int64_t S, int E);

/* Bytes of the GEMM tile plan moe_amd_permute() writes for S rows, E experts. */
size_t moe_amd_tile_plan_size(int64_t S, int E);

/* Counting sort of the flattened topk_index [S] by expert id.  Replaces the
 * sort / histc / cumsum of transformers/integrations/moe.py:389-403 (the
 * reference sort is unstable; this one is stable).  Outputs (int32):
 *   counts [E]            rows per expert (histc)
 *   offsets [E+1]         exclusive prefix of counts; offsets[E] = rows
 *                         owned by real experts (cumsum(counts)[-1])
 *   row_src [S]           sorted row r -> flat routed index t*K+k (perm)
 *   slot [S]              flat routed index -> sorted row (inverse perm)
 *   tile_plan             16-byte aligned, moe_amd_tile_plan_size() bytes:
 *                         int32 tile_starts[3][E+1] (exclusive prefix of
 *                         ceil(counts/BM), BM = 64, 128, 256), then per BM
 *                         an int4 table {expert, first row, end row, 0} of
 *                         every row tile; the grouped GEMMs read it. */
int moe_amd_permute(const int64_t* topk_index, int64_t S, int E, void* workspace,
                    size_t workspace_bytes, int32_t* counts, int32_t* offsets, int32_t* row_src,
                    int32_t* slot, void* tile_plan, size_t tile_plan_bytes, void* stream);

/* moe_amd_permute without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same outputs, bit for bit, as
 * moe_amd_permute; its scratch is a static device array of
 * MOE_PERMUTE_NOALLOC_SCRATCH_BYTES on each GPU (held until the process
 * ends), so it accepts only S, E with moe_amd_permute_workspace_size(S, E)
 * <= that size (e.g. E = 128 up to S of about 4.1 M routed rows) and
 * returns MOE_ERR_UNSUPPORTED beyond.  Calls that overlap on one GPU share
 * the array and race: order them (one stream, or events). */
enum { MOE_PERMUTE_NOALLOC_SCRATCH_BYTES = 8 << 20 };
int moe_amd_permute_noalloc(const int64_t* topk_index, int64_t S, int E, int32_t* counts,
                            int32_t* offsets, int32_t* row_src, int32_t* slot, void* tile_plan,
                            size_t tile_plan_bytes, void* stream);

/* ------------------------------------------------------- grouped GEMMs */
/* Grouped GEMMs: dtype MOE_DTYPE_BF16 (bf16 operands and results, fp32
 * accumulation on the bf16 MFMA) or, for the entry points without "fused"
 * or "gathered" in their name, MOE_DTYPE_F32 (fp32 operands and results on
 * the fp32 MFMA: the XS-standard layer's precision); the fused and gathered
 * backward entry points are bf16 only.  H and I must be multiples of 64;
 * pointers 16-byte aligned.
 * The expert of each row tile is read from the tile plan on the device, so
 * empty and skewed experts cost no host synchronisation.  The kernels are
 * persistent: one workgroup per compute unit walks a contiguous range of
 * tiles per XCD. */

/* gate_up = xs @ gate_up_proj[e]^T with xs[r] = hidden_states[row_src[r]/K],
 * then act = silu(gate) * up.  transformers/integrations/moe.py:439-447.
 * gate_up_out [S,2I] (may be NULL: inference), act_out [S,I]. */
int moe_amd_gemm_gate_up_swiglu(const void* hidden_states, const int32_t* row_src, int top_k,
                                const int32_t* offsets, const void* tile_plan,
                                const void* gate_up_proj, int64_t T, int64_t S, int E, int H,
                                int I, int dtype, void* gate_up_out, void* act_out,
                                void* stream);

/* y = act @ down_proj[e]^T.  transformers/integrations/moe.py:449-459.
 * y_out [S,H]. */
int moe_amd_gemm_down(const void* act, const int32_t* offsets, const void* tile_plan,
                      const void* down_proj, int64_t S, int E, int H, int I, int dtype,
                      void* y_out, void* stream);

/* Backward of GEMM-2 w.r.t. its input fused with the SwiGLU backward:
 * d_act = dy @ down_proj[e]; (d_gate, d_up) from gate_up; writes
 * d_gate_up [S,2I].  Autograd of integrations/moe.py:447,457 (formula :226-242).
 * With moe_amd_gemm_down_backward_dw and moe_amd_combine_backward this is
 * the unfused backward chain (from a materialised dy): the fp32 layer's
 * backward; in bf16 the layers take the fused pair below
 * (moe_amd_gemm_down_backward_dx_fused, _dw_gathered), and the bf16 forms
 * of these three serve callers that hold dy and the tests. */
int moe_amd_gemm_down_backward_dx_dswiglu(const void* dy, const int32_t* offsets,
                                          const void* tile_plan, const void* down_proj,
                                          const void* gate_up, int64_t S, int E, int H, int I,
                                          int dtype, void* d_gate_up, void* stream);

/* d_down_proj[e] = dy_e^T @ act_e  ([E,H,I]; zero for empty experts).
 * With a tile plan (may be null) the tiles are claimed from its dW schedule:
 * balanced under skewed routing; two dW launches that share one plan must
 * not run concurrently. */
int moe_amd_gemm_down_backward_dw(const void* dy, const void* act, const int32_t* offsets,
                                  const void* tile_plan, int64_t S, int E, int H, int I,
                                  int dtype, void* d_down_proj, void* stream);

/* The combine's backward fused into GEMM-2's backward, without the [S,H]
 * d_y = w * d_out[token] of moe_amd_combine_backward: per routed row r of
 * token t = row_src[r]/K, g = d_out[t] @ down_proj[e] (fp32 sums);
 * d_act = w[row_src[r]] * g and (d_gate, d_up) from gate_up as in
 * moe_amd_gemm_down_backward_dx_dswiglu -> d_gate_up [S,2I];
 * act_w [S,I] = w * act (act = silu(gate) * up recomputed from gate_up,
 * bitwise as the forward stored it), the input of
 * moe_amd_gemm_down_backward_dw_gathered; dw_partials
 * [T*K][moe_amd_gemm_down_backward_dx_fused_parts(I)] fp32: per 128
 * features, <g, act> over them = that block's share of
 * d_w[t,k] = <d_out[t], y[r]>, reduced by moe_amd_weight_grad_reduce.
 * topk_weights [T*K] in weights_dtype (fp32 or bf16).  Replaces the
 * autograd of transformers/integrations/moe.py:457-478 (weights multiply,
 * index_add) and of the down projection :449-459 (formula :226-242). */
int moe_amd_gemm_down_backward_dx_fused_parts(int I);
int moe_amd_gemm_down_backward_dx_fused(const void* d_out, const int32_t* row_src, int top_k,
                                        const int32_t* offsets, const void* tile_plan,
                                        const void* down_proj, const void* gate_up,
                                        const void* topk_weights, int weights_dtype, int64_t T,
                                        int64_t S, int E, int H, int I, int dtype,
                                        void* d_gate_up, void* act_w, float* dw_partials,
                                        void* stream);

/* d_down_proj[e] = sum over e's rows r of d_out[row_src[r]/K]^T act_w[r]
 * ([E,H,I]; zero for empty experts), d_out rows gathered through row_src:
 * with act_w = w * act this equals moe_amd_gemm_down_backward_dw on
 * d_y = w * d_out[token].  Tile plan as for moe_amd_gemm_down_backward_dw. */
int moe_amd_gemm_down_backward_dw_gathered(const void* d_out, const void* act_w,
                                           const int32_t* row_src, int top_k,
                                           const int32_t* offsets, const void* tile_plan,
                                           int64_t T, int64_t S, int E, int H, int I, int dtype,
                                           void* d_down_proj, void* stream);

/* Fused gradient accumulation of the two dW GEMMs: d_down_proj[e] +=
 * (moe_amd_gemm_down_backward_dw_gathered's d_down_proj[e]) and
 * d_gate_up_proj[e] += (moe_amd_gemm_gate_up_backward_dw's) in place, bf16
 * only, each element as torch adds two bf16 tensors (the GEMM result rounded
 * to bf16, added in fp32, rounded to nearest even): the bits autograd's
 * gradient accumulation gives.  Experts without routed rows are neither read
 * nor written.  The tile plan is required (its dW schedule lists those
 * experts last).  Replaces, for an expert bank shared by several layers
 * (src/models/global_moe.py:138, :147-151), each layer's dense dW tensor plus
 * the autograd accumulation that adds it to the bank's gradient (formula
 * transformers/integrations/moe.py:226-242). */
int moe_amd_gemm_down_backward_dw_gathered_accumulate(const void* d_out, const void* act_w,
                                                      const int32_t* row_src, int top_k,
                                                      const int32_t* offsets,
                                                      const void* tile_plan, int64_t T, int64_t S,
                                                      int E, int H, int I, int dtype,
                                                      void* d_down_proj, void* stream);
int moe_amd_gemm_gate_up_backward_dw_accumulate(const void* d_gate_up, const void* hidden_states,
                                                const int32_t* row_src, int top_k,
                                                const int32_t* offsets, const void* tile_plan,
                                                int64_t T, int64_t S, int E, int H, int I,
                                                int dtype, void* d_gate_up_proj, void* stream);

/* d_xs = d_gate_up @ gate_up_proj[e]  ([S,H]). */
int moe_amd_gemm_gate_up_backward_dx(const void* d_gate_up, const int32_t* offsets,
                                     const void* tile_plan, const void* gate_up_proj,
                                     int64_t S, int E, int H, int I, int dtype, void* d_xs,
                                     void* stream);

/* d_gate_up_proj[e] = d_gate_up_e^T @ xs_e, xs gathered from hidden_states
 * through row_src  ([E,2I,H]; zero for empty experts).  Tile plan as for
 * moe_amd_gemm_down_backward_dw. */
int moe_amd_gemm_gate_up_backward_dw(const void* d_gate_up, const void* hidden_states,
                                     const int32_t* row_src, int top_k, const int32_t* offsets,
                                     const void* tile_plan, int64_t T, int64_t S, int E, int H,
                                     int I, int dtype, void* d_gate_up_proj, void* stream);

/* ------------------------------------------------------------- combine */

/* out[t] = sum_k w[t,k] * y[slot[t*K+k]], accumulated in fp32 in k order,
 * rounded once to dtype; sentinel rows contribute zero.  With bf16 weights
 * each product is rounded to bf16 first (bf16 * bf16 in the reference).
 * transformers/integrations/moe.py:461-478. */
int moe_amd_combine(const void* y, const int32_t* slot, const int32_t* offsets,
                    const void* topk_weights, int weights_dtype, int64_t T, int K, int E, int H,
                    int dtype, void* out, void* stream);

/* Backward of the combine: d_y[slot[t,k]] = d_out[t] * w[t,k] (rounded to
 * dtype) and d_w[t,k] = <d_out[t], y[slot[t,k]]> (weights_dtype). */
int moe_amd_combine_backward(const void* d_out, const void* y, const int32_t* slot,
                             const int32_t* offsets, const void* topk_weights,
                             int weights_dtype, int64_t T, int K, int E, int H, int dtype,
                             void* d_y, void* d_topk_weights, void* stream);

/* d_topk_weights[i] = sum over c < n_part of partials[i*n_part + c] (fp32
 * in c order, rounded once to weights_dtype) for the T*K routed entries; 0
 * where slot[i] is a sentinel row.  The last step of the fused combine
 * backward (moe_amd_gemm_down_backward_dx_fused). */
int moe_amd_weight_grad_reduce(const float* partials, int n_part, const int32_t* slot,
                               const int32_t* offsets, int64_t T, int K, int E,
                               void* d_topk_weights, int weights_dtype, void* stream);

/* Backward of the gather xs = hidden_states[row_src // K]:
 * d_x[t] = sum_k d_xs[slot[t*K+k]] (fp32 accumulation, sentinels skipped). */
int moe_amd_gather_backward(const void* d_xs, const int32_t* slot, const int32_t* offsets,
                            int64_t T, int K, int E, int H, int dtype, void* d_x, void* stream);

/* The same plus a second gradient of the hidden states (the gating linear's,
 * when router and experts are one autograd node): d_x[t] =
 * dtype(dtype(sum_k d_xs[slot[t*K+k]]) + addend[t]), the rounding of
 * autograd accumulating two dtype-typed gradients of hidden_states.  No
 * counterpart in the reference, which adds the two gradients with a separate
 * elementwise kernel.  addend [T,H] in dtype. */
int moe_amd_gather_backward_add(const void* d_xs, const int32_t* slot, const int32_t* offsets,
                                const void* addend, int64_t T, int K, int E, int H, int dtype,
                                void* d_x, void* stream);

/* ---------------------------------------------------- routing consumers */

/* One pass over a layer's router probabilities probs [T,E] (fp32 or bf16):
 * counts[e] = sum over tokens of w[t] * (e among the token's top K) and
 * prob_sums[e] = sum_t w[t] * probs[t,e] (w = token_weights, or 1 when
 * null), margin[0] = sum_t (v_K - v_(K+1)) and margin[1] = min_t of it (the
 * K-th and (K+1)-th largest probabilities; 0 and +inf when K == E).  Output
 * in fp64, reduced in a fixed order (deterministic).  Replaces the
 * topk/one_hot/mean chains of src/models/load_balancing.py:45-88 and
 * src/utils/routing_stats.py:53-80, :143-191. */
size_t moe_amd_topk_stats_workspace_size(int64_t T, int E);
int moe_amd_topk_stats(const void* probs, int probs_dtype, const float* token_weights, int64_t T,
                       int E, int K, void* workspace, size_t workspace_bytes, double* counts,
                       double* prob_sums, double* margin, void* stream);

/* DeepSeek-V3 sequence-wise loss statistics of one layer (scores [T,E], T =
 * B sequences of S tokens): s' = s / (sum_e s + 1e-20) per token; counts[b,e]
 * = selections of e in sequence b (selected [T,K] int64 routed indices, or
 * the top K of s' when null) and mean_scores[b,e] = mean over the sequence
 * of s'[t,e] (fp64).  src/models/load_balancing.py:134-166. */
size_t moe_amd_seq_stats_workspace_size(int64_t T, int E, int B);
int moe_amd_seq_stats(const void* scores, int scores_dtype, const int64_t* selected, int64_t T,
                      int E, int K, int B, void* workspace, size_t workspace_bytes,
                      double* counts, double* mean_scores, void* stream);

/* Backward of the sequence-wise loss through the normalisation: with g[t,e]
 * = coef[b(t),e] the loss gradient w.r.t. s'[t,e], d_scores[t,e] =
 * (g[t,e] - sum_f g[t,f] s'[t,f]) / (sum_f s[t,f] + 1e-20), in scores'
 * dtype.  Autograd of load_balancing.py:143. */
int moe_amd_seq_aux_backward(const void* scores, int scores_dtype, const double* coef, int64_t T,
                             int E, int B, void* d_scores, void* stream);

/* Backward of the Switch loss: grad[t,e] = coef[e] * w[t] (w = 1 when
 * token_weights is null), in grad_dtype.  Autograd of load_balancing.py:87-88. */
int moe_amd_switch_aux_backward(const double* coef, const float* token_weights, int64_t T, int E,
                                int grad_dtype, void* grad, void* stream);

/* Aux-loss-free balancing step for L routers at once (train.py:79-139 without
 * the DDP all-reduce): counts[l] and biases[l] are device pointers to each
 * router's fp32 [E] local_tokens_per_expert and expert_bias (the two arrays
 * of L pointers live in device memory).  Per layer (is_global 0) bias +=
 * sign(mean(counts[l]) - counts[l]) * rate; pooled (is_global 1, alpha 0)
 * with the counts summed over layers; blended (alpha > 0) alpha * per-layer
 * + (1 - alpha) * pooled, in fp32 in the reference's operation order.
 * Counts are zeroed; stats = mean, unbiased std, min, max of all new biases
 * (fp64). */
int moe_amd_update_expert_biases(float* const* counts, float* const* biases, int L, int E,
                                 float update_rate, int is_global, double alpha, double* stats,
                                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_AMD_H */
