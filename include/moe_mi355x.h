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
 * stays torch's fp32 GEMM.
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
 * backward) and y [R,D]. D % 256 == 0, H % 256 == 0, E <= 1024. */
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

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
