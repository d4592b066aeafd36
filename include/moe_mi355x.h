/*
 * moe_mi355x.h — C ABI of libmoe_mi355x.so, the MI355X (gfx950) MoE-layer hot path.
 *
 * Conventions for every entry point:
 *   - all pointers are device pointers (HBM); bf16 tensors are passed as uint16_t*;
 *   - sizes are element counts; tensors are dense row-major (contiguous);
 *   - `stream` is a hipStream_t; work is enqueued on it and the call returns
 *     without synchronising;
 *   - nothing allocates: outputs and workspaces are supplied by the caller;
 *   - the return value is 0 on success or a negative MOE_ERR_* code.
 *
 * Shape symbols: N tokens, D model dim, E routed experts, K top-k, H expert
 * hidden dim, R = N*K routed rows.
 *
 * Routing limits taken together (router, histogram and reorder): E <= 512,
 * K <= 32. The grouped GEMMs take E <= 1024.
 *
 * Reference citations are to QIU023/torchtitan (file:line).
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* moe_stream_t; /* == hipStream_t */

#define MOE_OK 0
#define MOE_ERR_INVALID_ARGUMENT (-1)
#define MOE_ERR_UNSUPPORTED_SHAPE (-2)
#define MOE_ERR_LAUNCH (-3)
#define MOE_ERR_WORKSPACE (-4)

#define MOE_SCORE_SOFTMAX 0
#define MOE_SCORE_SIGMOID 1

/* element type of token rows for the permute / combine entry points */
#define MOE_DTYPE_BF16 0
#define MOE_DTYPE_FP32 1

/* Router after the gate GEMM: score function, + expert_bias for selection,
 * optional group-limited mask, top-k in torch.topk(sorted=False) GPU slot
 * order, gather of un-biased scores, route_norm, route_scale, and the debug
 * round-robin override.
 * Replaces TokenChoiceTopKRouter.forward, torchtitan/models/common/moe.py:211-266
 * (with _get_node_limited_routing_scores :169-209 and
 * _debug_force_load_balance_routing :152-167). The gate itself (moe.py:231-232)
 * is not here: the caller passes fp32 logits (the reference's fp32 GEMM under
 * autocast by default).
 * logits [N,E] fp32, expert_bias [E] fp32 or NULL -> scores [N,E] fp32 (saved
 * for backward), top_scores [N,K] fp32, selected_experts [N,K] int64.
 * n_expert_groups <= 0 disables group limiting. E <= 512, K <= 64. */
int moe_router_fwd(const float* logits, const float* expert_bias, int64_t n_tokens,
                   int32_t n_experts, int32_t top_k, int32_t score_func,
                   int32_t n_expert_groups, int32_t n_limited_groups, int32_t route_norm,
                   float route_scale, int32_t force_load_balance, float* scores,
                   float* top_scores, int64_t* selected_experts, moe_stream_t stream);

/* Autograd of moe.py:236-266: d(top_scores) -> d(logits) [N,E] fp32. */
int moe_router_bwd(const float* grad_top_scores, const float* scores,
                   const int64_t* selected_experts, int64_t n_tokens, int32_t n_experts,
                   int32_t top_k, int32_t score_func, int32_t route_norm, float route_scale,
                   float* grad_logits, moe_stream_t stream);

/* The gate's backward (autograd of the fp32 gate under autocast, moe.py:229-232)
 * on bf16 GEMMs: grad_logits [N,C] fp32 -> terms [N,3C] bf16 (hi | mid | lo),
 * hi = bf16(d), mid = bf16(d - hi), lo = bf16(d - hi - mid), so that
 * hi + mid + lo == d exactly and dx = terms.[W;W;W], dW = terms^T.x carry the
 * fp32 GEMMs' exact products. C % 4 == 0; both pointers 16-byte aligned. */
int moe_gate_grad_split3(const float* grad_logits, int64_t n_rows, int32_t n_cols, uint16_t* terms,
                         moe_stream_t stream);

/* grad_weight [E,D] bf16 from the fp32 partials [P,3E,D] of terms^T.x (P = 1, or
 * 2 token halves): t_b = p0_b (+ p1_b) for the hi, mid, lo row blocks b, then
 * bf16((t_hi + t_mid) + t_lo). D % 4 == 0; both pointers 16-byte aligned. */
int moe_gate_dw_reduce(const float* partials, int32_t n_parts, int32_t n_experts, int32_t dim,
                       uint16_t* grad_weight, moe_stream_t stream);

/* Shared expert SwiGLU between its GEMMs (feed_forward.py:53-54,
 * silu(w1 x) * w3 x): a1 = x.w1^T, a3 = x.w3^T [N,Hs] -> h = silu(a1) * a3,
 * silu's output rounded to the dtype before the product, as torch's two ops.
 * dtype MOE_DTYPE_BF16 or MOE_DTYPE_FP32 (16-byte chunks per thread when Hs is
 * a multiple of 8 resp. 4 elements and the pointers are 16-byte aligned, one
 * element per thread otherwise). */
int moe_swiglu_fwd(const void* a1, const void* a3, int64_t n_rows, int32_t hidden, int32_t dtype, void* h,
                   moe_stream_t stream);

/* Autograd of moe_swiglu_fwd: dh = dy.w2 [N,Hs] -> dgu [N,2Hs], dg =
 * silu_backward(dh * a3, a1) in columns [0,Hs) and du = dh * silu(a1) in [Hs,2Hs),
 * every op rounded as torch's; side by side so that [dW1; dW3] is one GEMM. */
int moe_swiglu_bwd(const void* dh, const void* a1, const void* a3, int64_t n_rows, int32_t hidden,
                   int32_t dtype, void* dgu, moe_stream_t stream);

/* Bytes of int32 workspace needed by moe_histogram / moe_reorder. */
int64_t moe_reorder_workspace_bytes(int64_t n_tokens, int32_t n_experts);

/* Tokens per expert: torch.histc(selected_experts, bins=E, min=0, max=E)
 * (moe.py:269-274) -> counts [E] int64; optionally offsets [E] int32 =
 * inclusive cumsum (moe.py:60). offsets may be NULL. */
int moe_histogram(const int64_t* selected_experts, int64_t n_tokens, int32_t top_k,
                  int32_t n_experts, void* workspace, int64_t workspace_bytes, int64_t* counts,
                  int32_t* offsets, moe_stream_t stream);

/* TokenReorderer.forward (moe.py:291-332): stable argsort of the flat expert
 * ids as a counting sort. Outputs: scores_sorted [R] fp32 (NULL to skip),
 * token_idx [R] int64, counts [E] int64, offsets [E] int32 (NULL to skip),
 * slot_pos [N,K] int32 (sorted position of token t's slot j), tok_pos [N,K]
 * int32 (token t's sorted positions, ascending). Precondition: each token's K
 * experts are distinct and in [0,E) (true for every router output). E <= 1024,
 * K <= 32. */
int moe_reorder(const int64_t* selected_experts, const float* top_scores, int64_t n_tokens,
                int32_t top_k, int32_t n_experts, void* workspace, int64_t workspace_bytes,
                float* scores_sorted, int64_t* token_idx, int64_t* counts, int32_t* offsets,
                int32_t* slot_pos, int32_t* tok_pos, moe_stream_t stream);

/* moe_reorder without a workspace argument. No counterpart in the reference:
 * for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). It allocates nothing: its workspace
 * is a fixed device array of MOE_REORDER_NOALLOC_SCRATCH_BYTES that each GPU
 * holds until the process ends, so 2 * ceil(N / 256) * E * 4 bytes must fit in
 * it (e.g. N <= 524288 tokens at E = 256), else MOE_ERR_WORKSPACE. All calls on
 * one GPU share that array: calls that overlap on one GPU (other streams or
 * threads) race. Outputs and arguments as moe_reorder. */
#define MOE_REORDER_NOALLOC_SCRATCH_BYTES (4 << 20)
int moe_reorder_noalloc(const int64_t* selected_experts, const float* top_scores, int64_t n_tokens,
                        int32_t top_k, int32_t n_experts, float* scores_sorted, int64_t* token_idx,
                        int64_t* counts, int32_t* offsets, int32_t* slot_pos, int32_t* tok_pos,
                        moe_stream_t stream);

/* Autograd of top_scores.view(-1)[perm] (moe.py:325): d(scores_sorted) [R] ->
 * d(top_scores) [N,K]. */
int moe_reorder_bwd(const float* grad_scores_sorted, const int32_t* slot_pos, int64_t n_tokens,
                    int32_t top_k, float* grad_top_scores, moe_stream_t stream);

/* routed_input = x[token_idx] and, if scores_sorted != NULL, the
 * score_before_experts scaling (t.float() * s).to(x.dtype) (moe.py:445-451).
 * x [N,D] (bf16 or fp32 per `dtype`) -> routed_input [R,D] of the same type.
 * D % 8 == 0 (bf16) or D % 4 == 0 (fp32). */
int moe_permute(const void* x, const int32_t* slot_pos, const float* scores_sorted,
                int64_t n_tokens, int32_t dim, int32_t top_k, int32_t dtype, void* routed_input,
                moe_stream_t stream);

/* Autograd of moe_permute: grad_routed [R,D] -> grad_x [N,D] (index backward,
 * accumulated in ascending sorted position; round_each=1 rounds to the row
 * type after every add, as ATen's index_put(accumulate=True) on row slices
 * does), and, when scores_sorted != NULL, grad_scores_sorted [R] = sum_d g*x. */
int moe_permute_bwd(const void* grad_routed, const void* x, const int32_t* tok_pos,
                    const float* scores_sorted, int64_t n_tokens, int32_t dim, int32_t top_k,
                    int32_t dtype, int32_t round_each, void* grad_x, float* grad_scores_sorted,
                    moe_stream_t stream);

/* out = deterministic_scatter_add(shared_out, token_idx, routed_output)
 * (torchtitan/ops/scatter_add.py:10-20, called at moe.py:471-475), with the
 * score_after scaling of moe.py:465-469 fused when scores_sorted != NULL.
 * shared_out [N,D] or NULL (zeros), routed_output [R,D] -> out [N,D].
 * Starting from shared_out[t], token t's K rows are added in ascending sorted
 * position with a rounding to the row type after every add (the order and
 * rounding of the reference's deterministic scatter_add on the GPU). */
int moe_combine(const void* shared_out, const void* routed_output, const int32_t* tok_pos,
                const float* scores_sorted, int64_t n_tokens, int32_t dim, int32_t top_k,
                int32_t dtype, void* out, moe_stream_t stream);

/* Autograd of moe_combine (scatter_add.py:28-33 plus the score_after
 * scaling): grad_out [N,D] -> grad_routed [R,D]; grad_scores_sorted [R] when
 * scores_sorted != NULL. The gradient of shared_out is grad_out itself. */
int moe_combine_bwd(const void* grad_out, const void* routed_output, const int32_t* slot_pos,
                    const int32_t* tok_pos, const float* scores_sorted, int64_t n_tokens,
                    int32_t dim, int32_t top_k, int32_t dtype, void* grad_routed,
                    float* grad_scores_sorted, moe_stream_t stream);

/* _run_experts_grouped_mm forward (moe.py:53-70): per expert segment,
 * g = x.w1^T, u = x.w3^T, h = silu(g)*u, y = h.w2^T, all bf16 with fp32
 * accumulation. counts [E] int64 (num_tokens_per_expert); x [R,D];
 * w1,w3 [E,H,D]; w2 [E,D,H]. Outputs g,u,h [R,H] (g,u,h saved for
 * backward) and y [R,D]. D % 64 == 0, H % 64 == 0, E <= 1024. */
int moe_grouped_swiglu_fwd(const uint16_t* x, const uint16_t* w1, const uint16_t* w2,
                           const uint16_t* w3, const int64_t* counts, int64_t n_rows,
                           int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* g,
                           uint16_t* u, uint16_t* h, uint16_t* y, moe_stream_t stream);

/* Autograd of _run_experts_grouped_mm (the three torch._grouped_mm backward
 * passes plus SwiGLU backward): dy [R,D] -> dx [R,D], dw1,dw3 [E,H,D],
 * dw2 [E,D,H] (experts with no tokens get zero gradients).
 * dgu_workspace is [R, 2H] bf16. Runs the four backward kernels below in
 * order. */
int moe_grouped_swiglu_bwd(const uint16_t* dy, const uint16_t* x, const uint16_t* w1,
                           const uint16_t* w2, const uint16_t* w3, const int64_t* counts,
                           const uint16_t* g, const uint16_t* u, const uint16_t* h,
                           int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                           uint16_t* dgu_workspace, uint16_t* dx, uint16_t* dw1, uint16_t* dw2,
                           uint16_t* dw3, moe_stream_t stream);

/* The grouped GEMM kernels one at a time (each is one launch). Same shapes and
 * conventions as moe_grouped_swiglu_fwd / _bwd above.
 *
 * gate_up: the first two torch._grouped_mm of moe.py:62-67 fused with SwiGLU:
 *   g = x.w1^T, u = x.w3^T, h = bf16(bf16(silu(g)) * u). */
int moe_grouped_gemm_gate_up(const uint16_t* x, const uint16_t* w1, const uint16_t* w3,
                             const int64_t* counts, int64_t n_rows, int32_t n_experts,
                             int32_t dim, int32_t hidden, uint16_t* g, uint16_t* u, uint16_t* h,
                             moe_stream_t stream);
/* down: y = h.w2^T (moe.py:68). */
int moe_grouped_gemm_down(const uint16_t* h, const uint16_t* w2, const int64_t* counts,
                          int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                          uint16_t* y, moe_stream_t stream);
/* bwd_dgu: dh = dy.w2 (grad of moe.py:68 w.r.t. h) and the SwiGLU backward:
 * dgu [R,2H] = [dg | du]. */
int moe_grouped_gemm_bwd_dgu(const uint16_t* dy, const uint16_t* w2, const uint16_t* g,
                             const uint16_t* u, const int64_t* counts, int64_t n_rows,
                             int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* dgu,
                             moe_stream_t stream);
/* bwd_dx: dx = dg.w1 + du.w3 (one GEMM over the concatenated 2H axis). */
int moe_grouped_gemm_bwd_dx(const uint16_t* dgu, const uint16_t* w1, const uint16_t* w3,
                            const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                            int32_t hidden, uint16_t* dx, moe_stream_t stream);
/* bwd_dw13: dw1[e] = dg_e^T.x_e, dw3[e] = du_e^T.x_e (zeros for empty experts). */
int moe_grouped_gemm_bwd_dw13(const uint16_t* dgu, const uint16_t* x, const int64_t* counts,
                              int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                              uint16_t* dw1, uint16_t* dw3, moe_stream_t stream);
/* bwd_dw2: dw2[e] = dy_e^T.h_e (zeros for empty experts). */
int moe_grouped_gemm_bwd_dw2(const uint16_t* dy, const uint16_t* h, const int64_t* counts,
                             int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                             uint16_t* dw2, moe_stream_t stream);
/* No counterpart in the reference; for tests: the pointwise arithmetic of the
 * gate_up and bwd_dgu SwiGLU epilogues on its own. For bf16 g[0..n), writes fp32
 * silu[i] = g/(1+exp(-g)) and sigmoid[i] = 1/(1+exp(-g)) exactly as those
 * epilogues compute them before rounding (a pair 2i, 2i+1 takes the fast form
 * when both lie in its range, as a block of the epilogues does), so that they can
 * be compared with torch's silu and sigmoid over every bf16 value. */
int moe_swiglu_pointwise_f32(const uint16_t* g, float* silu, float* sigmoid, int64_t n,
                             moe_stream_t stream);

/* ---- fp32 experts: _run_experts_for_loop in the input dtype --------------
 * Replace the per-expert fp32 matmuls of torchtitan/models/common/moe.py:24-50
 * (and their autograd) with one launch per GEMM over all experts: fp32
 * operands, fp32 accumulation (v_mfma_f32_16x16x4f32), the SwiGLU of :41-43 in
 * fp32. Same layouts as the bf16 entry points, fp32 elements; D, H multiples of
 * 64, E <= 1024; rows past sum(counts) are not written. */

/* g = x w1^T, u = x w3^T, h = silu(g) * u per expert segment (moe.py:41-42). */
int moe_grouped_gemm_f32_gate_up(const float* x, const float* w1, const float* w3, const int64_t* counts,
                                 int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden, float* g,
                                 float* u, float* h, moe_stream_t stream);

/* y = h w2^T per expert segment (moe.py:43). */
int moe_grouped_gemm_f32_down(const float* h, const float* w2, const int64_t* counts, int64_t n_rows,
                              int32_t n_experts, int32_t dim, int32_t hidden, float* y, moe_stream_t stream);

/* Autograd of moe.py:41-43 through h: dh = dy w2; du = dh * silu(g);
 * dg = (dh * u) * sigmoid(g) (1 + g (1 - sigmoid(g))). dg, du [R, H]. */
int moe_grouped_gemm_f32_bwd_dgu(const float* dy, const float* w2, const float* g, const float* u,
                                 const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                 int32_t hidden, float* dg, float* du, moe_stream_t stream);

/* dx = dg w1 + du w3 per expert segment (autograd of moe.py:41-42). */
int moe_grouped_gemm_f32_bwd_dx(const float* dg, const float* du, const float* w1, const float* w3,
                                const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                int32_t hidden, float* dx, moe_stream_t stream);

/* Weight gradient out[e] = a_e^T b_e over expert e's rows: a [R, m], b [R, n]
 * -> out [E, m, n] (dw1 = dg^T x, dw3 = du^T x, dw2 = dy^T h; zero for empty
 * experts). m, n multiples of 64. */
int moe_grouped_gemm_f32_bwd_dw(const float* a, const float* b, const int64_t* counts, int64_t n_rows,
                                int32_t n_experts, int32_t m, int32_t n, float* out, moe_stream_t stream);

/* ---------------------------------------------------------------------------
 * gpt-oss experts (torchtitan/models/gpt_oss/moe.py:43-52, 92-122, the
 * grouped-mm path): mlp1_weight [E, 2H, D] bf16 with the glu row 2j and the
 * linear row 2j + 1, mlp1_bias [E, 2H], mlp2_weight [E, D, H], mlp2_bias
 * [E, D] (biases bf16). Forward, every op rounded to bf16:
 *   h1 = bf16(x . mlp1^T) + mlp1_bias;  g = h1[:, 0::2], u = h1[:, 1::2]
 *   h  = (clamp(g, max=L) * sigmoid(1.702 clamp(g, max=L))) * (clamp(u, -L, L) + 1)
 *   y  = bf16(h . mlp2^T) + mlp2_bias
 * with L = swiglu_limit rounded to bf16. D % 64 == 0, H % 64 == 0.
 * ------------------------------------------------------------------------- */

/* g, u, h [R, H] (g, u = the biased pre-clamp halves, saved for backward). */
int moe_grouped_gemm_oss_gate_up(const uint16_t* x, const uint16_t* mlp1_weight, const uint16_t* mlp1_bias,
                                 const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                 int32_t hidden, float swiglu_limit, uint16_t* g, uint16_t* u, uint16_t* h,
                                 moe_stream_t stream);
/* y [R, D] = bf16(h . mlp2^T) + mlp2_bias. */
int moe_grouped_gemm_oss_down(const uint16_t* h, const uint16_t* mlp2_weight, const uint16_t* mlp2_bias,
                              const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                              int32_t hidden, uint16_t* y, moe_stream_t stream);
/* dh = bf16(dy . mlp2), then the autograd of the clamped SwiGLU (each bf16 op's
 * gradient rounded to bf16, clamp gradients zero outside the limits):
 * dgu [R, 2H] = [dg | du] (the gradients of the glu and linear halves of h1). */
int moe_grouped_gemm_oss_bwd_dgu(const uint16_t* dy, const uint16_t* mlp2_weight, const uint16_t* g,
                                 const uint16_t* u, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                 int32_t dim, int32_t hidden, float swiglu_limit, uint16_t* dgu,
                                 moe_stream_t stream);
/* dx [R, D] = dh1 . mlp1 (one fp32 accumulation over 2H, rounded once). */
int moe_grouped_gemm_oss_bwd_dx(const uint16_t* dgu, const uint16_t* mlp1_weight, const int64_t* counts,
                                int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* dx,
                                moe_stream_t stream);
/* dmlp1_weight [E, 2H, D] = dh1_e^T . x_e, glu / linear rows interleaved (zeros
 * for empty experts). dmlp2_weight is moe_grouped_gemm_bwd_dw2 (same layout as w2). */
int moe_grouped_gemm_oss_bwd_dw1(const uint16_t* dgu, const uint16_t* x, const int64_t* counts,
                                 int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                                 uint16_t* dmlp1_weight, moe_stream_t stream);
/* Bias gradients (the backward of bias.repeat_interleave(counts)): per expert e
 * and column c < cols, out[e*ld_out + c*col_stride] = sum over the expert's rows
 * r of src[r*ld_src + c], fp32 in a fixed order. src bf16, cols % 64 == 0,
 * ld_src % 8 == 0. */
int moe_grouped_col_sum(const uint16_t* src, int64_t ld_src, const int64_t* counts, int64_t n_rows,
                        int32_t n_experts, int32_t cols, float* out, int64_t ld_out, int32_t col_stride,
                        moe_stream_t stream);

/* ---------------------------------------------------------------------------
 * fp8 e4m3 (OCP e4m3fn) grouped SwiGLU experts. The reference's fp8 path is
 * torchao's Float8TrainingOpConfig on the experts
 * (torchtitan/components/quantization/float8.py:260-288): dynamic rowwise
 * scales, fp32 accumulation, bf16 outputs, token groups padded to 16
 * (quantization/__init__.py:37-40). Quantization with torchao's power-of-two
 * scales: s = 2^-j, j = floor(log2(fp32(448 / max(amax, 1e-12)))) (the division
 * in fp64), q = e4m3fn(x / s) rounded to nearest even (x / s exact, |x / s| <= 448).
 * fp8 tensors are uint8_t*.
 * ------------------------------------------------------------------------- */

/* Rows of the token-transposed fp8 tensors: n_rows + n_experts * 127 (every
 * group starts at a multiple of 128); round it up to a multiple of 128. With
 * 128-byte aligned tensors every row of those tensors, and every group in it,
 * starts on a 128-byte line, so the transposing quantizers and the weight-gradient
 * GEMMs read and write whole lines, with no partly empty first pass or k-step. */
int64_t moe_fp8_padded_rows(int64_t n_rows, int32_t n_experts);

/* x [rows, cols] bf16 -> q [rows, cols] fp8, scale [rows] (one per row). */
int moe_fp8_quant_rows(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q, float* scale,
                       moe_stream_t stream);

/* x [E, a, b] bf16 -> per expert e and column j: scale[e*scale_expert_stride + j]
 * = the scale of the amax over a, and the quantized column written as a row of a values
 * at q + e*q_expert_stride + j*q_row_stride (a transposed copy). */
int moe_fp8_quant_cols_t(const uint16_t* x, int32_t n_experts, int32_t a, int32_t b, uint8_t* q,
                         int64_t q_expert_stride, int64_t q_row_stride, float* scale,
                         int64_t scale_expert_stride, moe_stream_t stream);

/* moe_fp8_quant_cols_t with the column amax [E, b] already known (from
 * moe_fp8_quant_rows_colamax of the same x): x is read once. */
int moe_fp8_quant_cols_t_amax(const uint16_t* x, const float* col_amax, int32_t n_experts, int32_t a,
                              int32_t b, uint8_t* q, int64_t q_expert_stride, int64_t q_row_stride,
                              float* scale, int64_t scale_expert_stride, moe_stream_t stream);

/* The weights' two rowwise quantizations (torchao's float8 grouped GEMM quantizes
 * each weight along the forward's and the backward's contraction,
 * quantization/float8.py:260-288) from two reads instead of three: x [E, a, b]
 * bf16 -> q [E, a, b] fp8 with one scale per row (as moe_fp8_quant_rows over b),
 * and col_amax [E, b] = the amax over a of each column (NaN ignored), max-
 * accumulated: the caller zeroes it. b % 8 == 0, b <= 8192. */
int moe_fp8_quant_rows_colamax(const uint16_t* x, int32_t n_experts, int32_t a, int32_t b, uint8_t* q,
                               float* scale, float* col_amax, moe_stream_t stream);

/* x [n_rows, cols] bf16 in expert token groups (counts) -> q [cols, padded_rows]
 * fp8 with group e at the 128-aligned offset sum_{e'<e} ceil128(count_e') and
 * zero padding up to ceil128(count_e); scale [E, cols] over the group's tokens
 * (not written for empty groups). */
int moe_fp8_quant_tokens_t(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                           int32_t cols, int64_t padded_rows, uint8_t* q, float* scale,
                           moe_stream_t stream);

/* moe_fp8_quant_tokens_t with each group's column amax [E, cols] already known
 * (from moe_fp8_quant_rows_groupamax of the same x): x is read once. */
int moe_fp8_quant_tokens_t_amax(const uint16_t* x, const float* group_amax, const int64_t* counts,
                                int64_t n_rows, int32_t n_experts, int32_t cols, int64_t padded_rows,
                                uint8_t* q, float* scale, moe_stream_t stream);

/* The token operands' two rowwise quantizations (torchao's float8 grouped GEMM
 * quantizes the routed tokens, their gradient and the SwiGLU intermediates along
 * each GEMM's contraction, quantization/float8.py:260-288) from two reads instead
 * of three: x [n_rows, cols] bf16 in expert token groups (counts) -> q [n_rows,
 * cols] fp8 with one scale per row piece (as moe_fp8_quant_rows over cols /
 * pieces columns: scale[r * pieces + p], pieces 1 or 2), and group_amax [E, cols]
 * = the amax of each column over each group's rows (NaN ignored), max-
 * accumulated: the caller zeroes it. Rows past the last group are quantized
 * but enter no amax. cols % (8 * pieces) == 0, cols <= 8192. */
int moe_fp8_quant_rows_groupamax(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                 int32_t cols, int32_t pieces, uint8_t* q, float* scale, float* group_amax,
                                 moe_stream_t stream);

/* moe_fp8_quant_rows_groupamax (pieces = 1) and moe_fp8_quant_tokens_t_amax of the
 * routed rows x[token_idx[r]] (times row_scale[r], rounded to bf16, when row_scale
 * != NULL) read from src [n_src, cols] in place: the expert permute (moe.py:445-451,
 * x[token_idx] * score) and the fp8 quantizations of its output without writing
 * the routed rows. Rows whose index is outside [0, n_src) read as zeros. n_src >= 1;
 * src 16-byte aligned. */
int moe_fp8_quant_rows_groupamax_gather(const uint16_t* src, int64_t n_src, const int64_t* token_idx,
                                        const float* row_scale, const int64_t* counts, int64_t n_rows,
                                        int32_t n_experts, int32_t cols, uint8_t* q, float* scale,
                                        float* group_amax, moe_stream_t stream);
int moe_fp8_quant_tokens_t_amax_gather(const uint16_t* src, int64_t n_src, const int64_t* token_idx,
                                       const float* row_scale, const float* group_amax, const int64_t* counts,
                                       int64_t n_rows, int32_t n_experts, int32_t cols, int64_t padded_rows,
                                       uint8_t* q, float* scale, moe_stream_t stream);

/* fp8 forward of _run_experts_grouped_mm (moe.py:62-67): g = (qx.qw1^T)*sx*sw1,
 * u likewise with w3, h = bf16(bf16(silu(g)) * u). sw1, sw3 [E, H]. */
int moe_fp8_gemm_gate_up(const uint8_t* qx, const float* sx, const uint8_t* qw1, const float* sw1,
                         const uint8_t* qw3, const float* sw3, const int64_t* counts, int64_t n_rows,
                         int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* g, uint16_t* u,
                         uint16_t* h, moe_stream_t stream);
/* fp8 y = (qh.qw2^T)*sh*sw2 (moe.py:68); sw2 [E, D]. */
int moe_fp8_gemm_down(const uint8_t* qh, const float* sh, const uint8_t* qw2, const float* sw2,
                      const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                      uint16_t* y, moe_stream_t stream);
/* fp8 dh = (qdy.qw2t^T)*sdy*sw2t with qw2t [E, H, D] (w2 quantized along D),
 * then the SwiGLU backward -> dgu [R, 2H] bf16. */
int moe_fp8_gemm_bwd_dgu(const uint8_t* qdy, const float* sdy, const uint8_t* qw2t, const float* sw2t,
                         const uint16_t* g, const uint16_t* u, const int64_t* counts, int64_t n_rows,
                         int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* dgu, moe_stream_t stream);
/* fp8 dx = bf16(dg.w1 scaled) + bf16(du.w3 scaled): qdgu [R, 2H] with sdgu [R, 2]
 * (one scale per half), qw13t [E, D, 2H] with sw13t [E, 2, D]. */
int moe_fp8_gemm_bwd_dx(const uint8_t* qdgu, const float* sdgu, const uint8_t* qw13t, const float* sw13t,
                        const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                        uint16_t* dx, moe_stream_t stream);
/* fp8 dw1[e], dw3[e] = dgu_e^T . x_e from the token-transposed fp8 tensors
 * qdgut [2H, padded_rows] (sdgut [E, 2H]) and qxt [D, padded_rows] (sxt [E, D]);
 * experts without tokens get zeros. */
int moe_fp8_gemm_bwd_dw13(const uint8_t* qdgut, const float* sdgut, const uint8_t* qxt, const float* sxt,
                          const int64_t* counts, int64_t n_rows, int64_t padded_rows, int32_t n_experts,
                          int32_t dim, int32_t hidden, uint16_t* dw1, uint16_t* dw3, moe_stream_t stream);
/* fp8 dw2[e] = dy_e^T . h_e from qdyt [D, padded_rows] (sdyt [E, D]) and
 * qht [H, padded_rows] (sht [E, H]). */
int moe_fp8_gemm_bwd_dw2(const uint8_t* qdyt, const float* sdyt, const uint8_t* qht, const float* sht,
                         const int64_t* counts, int64_t n_rows, int64_t padded_rows, int32_t n_experts,
                         int32_t dim, int32_t hidden, uint16_t* dw2, moe_stream_t stream);

/* ---------------------------------------------------------------------------
 * MXFP8 grouped SwiGLU experts: torchao's MXFP8TrainingOpConfig with recipe
 * "mxfp8_rceil", applied by MXFP8Converter
 * (torchtitan/components/quantization/mx.py:25-128), token groups padded to
 * 32 (quantization/__init__.py:36-40). Every row is quantized in blocks of
 * 32 consecutive elements along the contraction: e8m0 scale byte
 * e = clamp(ceil(log2(amax / 448)), -127, 127) + 127 (255 for NaN), elements
 * e4m3fn(clamp(x * 2^(127 - e), +-448)) (x * 1 when e == 0). The GEMMs apply
 * both scales in the MFMA (fp32 accumulation, bf16 outputs). Scales of
 * row-quantized tensors are [rows, cols / 32]; of token-transposed ones
 * k-block major, [padded_rows / 32, cols].
 * ------------------------------------------------------------------------- */

/* Rows of the token-transposed MXFP8 tensors: n_rows + n_experts * 127 rounded
 * up to a multiple of 128 (every group starts at a multiple of 128, as for
 * moe_fp8_padded_rows). */
int64_t moe_mxfp8_padded_rows(int64_t n_rows, int32_t n_experts);

/* x [rows, cols] bf16 (cols % 32 == 0) -> q [rows, cols], scale [rows, cols / 32]. */
int moe_mxfp8_quant_rows(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q, uint8_t* scale,
                         moe_stream_t stream);

/* x [E, a, b] bf16 -> per expert e and column j the column quantized along a
 * (blocks of 32) and written as a row of a values at
 * q + e*q_expert_stride + j*q_row_stride, its a / 32 scales at
 * scale + e*scale_expert_stride + j*scale_row_stride. */
int moe_mxfp8_quant_cols_t(const uint16_t* x, int32_t n_experts, int32_t a, int32_t b, uint8_t* q,
                           int64_t q_expert_stride, int64_t q_row_stride, uint8_t* scale,
                           int64_t scale_expert_stride, int64_t scale_row_stride, moe_stream_t stream);

/* x [n_rows, cols] bf16 in expert token groups -> q [cols, padded_rows] with
 * group e at the 128-aligned offset sum_{e'<e} ceil128(count_e') (zero padded),
 * quantized along the tokens in blocks of 32; scale [padded_rows / 32, cols]
 * (blocks of empty groups and past the groups are not written). */
int moe_mxfp8_quant_tokens_t(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                             int32_t cols, int64_t padded_rows, uint8_t* q, uint8_t* scale,
                             moe_stream_t stream);

/* Both MX layouts from one read of x [E, a, b] (weights): q_rows [E, a, b] with
 * scale_rows [E, a, b/32] (as moe_mxfp8_quant_rows on [E*a, b]) and the
 * transposed layout of moe_mxfp8_quant_cols_t (same strides). */
int moe_mxfp8_quant_dual_cols(const uint16_t* x, int32_t n_experts, int32_t a, int32_t b, uint8_t* q_rows,
                              uint8_t* scale_rows, uint8_t* q, int64_t q_expert_stride, int64_t q_row_stride,
                              uint8_t* scale, int64_t scale_expert_stride, int64_t scale_row_stride,
                              moe_stream_t stream);
/* Both MX layouts from one read of x [n_rows, cols] in token groups: q_rows
 * [n_rows, cols] with scale_rows [n_rows, cols/32] for the rows of the groups,
 * and the token-transposed layout of moe_mxfp8_quant_tokens_t. */
int moe_mxfp8_quant_dual_tokens(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                int32_t cols, int64_t padded_rows, uint8_t* q_rows, uint8_t* scale_rows,
                                uint8_t* q, uint8_t* scale, moe_stream_t stream);

/* moe_mxfp8_quant_dual_tokens of the routed rows x[token_idx[r]] (times
 * row_scale[r], rounded to bf16, when row_scale != NULL) read from src [n_src,
 * cols] in place: the expert permute (moe.py:445-451, x[token_idx] * score) and
 * the quantization of its output in one pass, without writing the routed rows.
 * Rows whose index is outside [0, n_src) read as zeros. n_src >= 1; src must be 16-byte
 * aligned (rows are read in 16-byte pieces). */
int moe_mxfp8_quant_dual_tokens_gather(const uint16_t* src, int64_t n_src, const int64_t* token_idx,
                                       const float* row_scale, const int64_t* counts, int64_t n_rows,
                                       int32_t n_experts, int32_t cols, int64_t padded_rows, uint8_t* q_rows,
                                       uint8_t* scale_rows, uint8_t* q, uint8_t* scale, moe_stream_t stream);

/* MXFP8 g, u, h as moe_fp8_gemm_gate_up; sx [R, D/32], sw1 and sw3 [E, H, D/32]. */
int moe_mxfp8_gemm_gate_up(const uint8_t* qx, const uint8_t* sx, const uint8_t* qw1, const uint8_t* sw1,
                           const uint8_t* qw3, const uint8_t* sw3, const int64_t* counts, int64_t n_rows,
                           int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* g, uint16_t* u,
                           uint16_t* h, moe_stream_t stream);
/* MXFP8 y = qh.qw2^T; sh [R, H/32], sw2 [E, D, H/32]. */
int moe_mxfp8_gemm_down(const uint8_t* qh, const uint8_t* sh, const uint8_t* qw2, const uint8_t* sw2,
                        const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                        uint16_t* y, moe_stream_t stream);
/* MXFP8 dh = qdy.qw2t^T (sdy [R, D/32], qw2t [E, H, D], sw2t [E, H, D/32]),
 * then the SwiGLU backward -> dgu [R, 2H] bf16. */
int moe_mxfp8_gemm_bwd_dgu(const uint8_t* qdy, const uint8_t* sdy, const uint8_t* qw2t, const uint8_t* sw2t,
                           const uint16_t* g, const uint16_t* u, const int64_t* counts, int64_t n_rows,
                           int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* dgu, moe_stream_t stream);
/* MXFP8 dx = bf16(dg.w1) + bf16(du.w3): qdgu [R, 2H] with sdgu [R, 2H/32],
 * qw13t [E, D, 2H] with sw13t [E, D, 2H/32] (w1 half first). */
int moe_mxfp8_gemm_bwd_dx(const uint8_t* qdgu, const uint8_t* sdgu, const uint8_t* qw13t, const uint8_t* sw13t,
                          const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                          uint16_t* dx, moe_stream_t stream);
/* MXFP8 dw1[e], dw3[e] = dgu_e^T . x_e from qdgut [2H, padded_rows]
 * (sdgut [padded_rows/32, 2H]) and qxt [D, padded_rows] (sxt [padded_rows/32, D]). */
int moe_mxfp8_gemm_bwd_dw13(const uint8_t* qdgut, const uint8_t* sdgut, const uint8_t* qxt, const uint8_t* sxt,
                            const int64_t* counts, int64_t n_rows, int64_t padded_rows, int32_t n_experts,
                            int32_t dim, int32_t hidden, uint16_t* dw1, uint16_t* dw3, moe_stream_t stream);
/* MXFP8 dw2[e] = dy_e^T . h_e from qdyt [D, padded_rows] (sdyt [padded_rows/32, D])
 * and qht [H, padded_rows] (sht [padded_rows/32, H]). */
int moe_mxfp8_gemm_bwd_dw2(const uint8_t* qdyt, const uint8_t* sdyt, const uint8_t* qht, const uint8_t* sht,
                           const int64_t* counts, int64_t n_rows, int64_t padded_rows, int32_t n_experts,
                           int32_t dim, int32_t hidden, uint16_t* dw2, moe_stream_t stream);

/* ---- auxiliary-loss-free load balancing (optimizer step pre-hook) ---- */

/* For every MoE layer l < n_layers (<= 64), with t = tokens_per_expert[l]
 * ([E] fp32, integer-valued; floor(t / 2) first when halve[l], the blocks that
 * recompute their forward): expert_bias[l] += d - mean(d) with
 * d = coeff[l] * sign(mean(t) - t); then tokens_per_expert[l] = 0.
 * tokens_per_expert, expert_bias, coeff and halve are HOST arrays (the first
 * two of device pointers). E <= 1024. One launch for all layers.
 * Replaces _update_expert_bias of register_moe_load_balancing_hook,
 * torchtitan/components/optimizer.py:366-437 (the count all-reduce at
 * :400-414 belongs to the caller). */
int moe_expert_bias_update(float* const* tokens_per_expert, float* const* expert_bias, const float* coeff,
                           const int32_t* halve, int32_t n_layers, int32_t n_experts, moe_stream_t stream);

/* ---- expert parallelism: rank-major -> expert-major local permute ---- */

/* tokens_per_expert_group [num_ranks * experts_per_rank] int64 (rank-major)
 * -> permuted_indices [total] int64: output row p of the expert-major layout
 * reads input row permuted_indices[p]; num_tokens_per_expert [experts_per_rank]
 * int64 (nullable) = the counts summed over ranks. total is the number of
 * received rows (the sum of the counts, known to the caller from the
 * all-to-all splits); positions past that sum get -1.
 * num_ranks * experts_per_rank <= 2048.
 * Replaces _generate_permute_indices, torchtitan/distributed/expert_parallel.py:26-67. */
int moe_ep_permute_indices(const int64_t* tokens_per_expert_group, int32_t experts_per_rank, int32_t num_ranks,
                           int64_t total, int64_t* permuted_indices, int64_t* num_tokens_per_expert,
                           moe_stream_t stream);
/* The permute of moe_ep_permute_indices with every expert's group padded by
 * zero rows to a multiple of pad_multiple (16 for fp8, 32 for MXFP8): padding
 * positions get index sum(counts) (a zero row appended after the input rows),
 * padded_tokens_per_expert [experts_per_rank] int64 (nullable) the padded group
 * sizes and group_offsets [experts_per_rank] int32 (nullable) their inclusive
 * ends; total_padded = the sum of the padded sizes.
 * Replaces torchao's permute_and_pad as called by TorchAOExpertParallel,
 * torchtitan/distributed/expert_parallel.py:537-551. */
int moe_ep_permute_pad_indices(const int64_t* tokens_per_expert_group, int32_t experts_per_rank, int32_t num_ranks,
                               int32_t pad_multiple, int64_t total_padded, int64_t* permuted_indices,
                               int64_t* padded_tokens_per_expert, int32_t* group_offsets, moe_stream_t stream);
/* dst[i, :] = src[idx[i], :] for i < n_rows; idx == n_src_rows writes a zero row
 * (the appended padding row); rows with other idx outside [0, n_src_rows) are
 * left untouched. Rows of `dim` elements of `dtype` (MOE_DTYPE_*), 16-byte
 * multiples. Replaces x[permuted_indices, :] of _permute, expert_parallel.py:70-74. */
int moe_gather_rows(const void* src, int64_t n_src_rows, const int64_t* idx, int64_t n_rows, int32_t dim,
                    int32_t dtype, void* dst, moe_stream_t stream);
/* dst[idx[i], :] = src[i, :] (idx a permutation; rows with idx outside
 * [0, n_dst_rows) are skipped). Replaces out_unpermuted[permuted_indices, :] = out
 * of _unpermute, expert_parallel.py:77-80. */
int moe_scatter_rows(const void* src, const int64_t* idx, int64_t n_rows, int32_t dim, int32_t dtype, void* dst,
                     int64_t n_dst_rows, moe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
