"""torch.library custom ops over the MI355X MoE kernels (namespace ``moe_mi355x``).

Each op is a thin host wrapper around one C-ABI entry point of
``libmoe_mi355x.so``: it allocates outputs and workspaces with torch's caching
allocator, passes raw device pointers and torch's current stream, and maps
status codes to exceptions. Every op has a fake (meta) implementation so it
stays opaque under ``torch.compile``, and an autograd formula, following the
registration pattern of torchtitan/ops/scatter_add.py:10-48.

There is no CPU or eager-torch fallback: the ops raise on non-GPU tensors and
when the library is missing.
"""

from __future__ import annotations

import torch
from torch import Tensor

from ._lib import call, lib, ptr, require_gpu, stream_of

SCORE_FUNCS = {"softmax": 0, "sigmoid": 1}
# Shape limits of the routing kernels taken together: the router takes E <= 512
# and K <= 64, the histogram and reorder K <= 32 (and E <= 1024).
MAX_EXPERTS = 512
MAX_TOP_K = 32
DTYPE_CODES = {torch.bfloat16: 0, torch.float32: 1}

# Gradient of x[token_idx] accumulates a token's K rows with a rounding to the
# row dtype after each add, as ATen's index_put(accumulate=True) kernel does for
# row slices on the GPU.
PERMUTE_BWD_ROUND_EACH = True


def _dtype_code(t: Tensor) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"MoE row kernels support bfloat16 and float32 rows, got {t.dtype}") from None


def _workspace(n_tokens: int, num_experts: int, device: torch.device) -> Tensor:
    nbytes = lib().moe_reorder_workspace_bytes(n_tokens, num_experts)
    return torch.empty(max(nbytes, 4), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# router: score function, bias, group limit, top-k, gather, norm, scale
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::router", mutates_args=())
def router(
    logits: Tensor,
    expert_bias: Tensor | None,
    num_experts: int,
    top_k: int,
    score_func: int,
    num_expert_groups: int,
    num_limited_groups: int,
    route_norm: bool,
    route_scale: float,
    force_load_balance: bool,
    with_counts: bool = True,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Returns (top_scores [N,K] f32, selected_experts [N,K] i64, counts [E] i64, scores [N,E] f32).
    with_counts=False skips the histogram (moe.py:269-274) and returns an empty counts
    tensor, for callers that take the counts from the reorder that follows (its own
    histogram, moe.py:312-317, the same counts on one GPU)."""
    require_gpu(logits, expert_bias)
    logits = logits.float().contiguous()
    n = logits.shape[0]
    dev = logits.device
    bias = expert_bias.float().contiguous() if expert_bias is not None else None
    scores = torch.empty_like(logits)
    top_scores = torch.empty(n, top_k, dtype=torch.float32, device=dev)
    idx = torch.empty(n, top_k, dtype=torch.int64, device=dev)
    counts = torch.empty(num_experts if with_counts else 0, dtype=torch.int64, device=dev)
    s = stream_of(logits)
    call(
        "moe_router_fwd", ptr(logits), ptr(bias), n, num_experts, top_k, score_func, num_expert_groups,
            num_limited_groups, int(route_norm), route_scale, int(force_load_balance),
            ptr(scores), ptr(top_scores), ptr(idx), s,
    )
    if with_counts:
        ws = _workspace(n, num_experts, dev)
        call(
            "moe_histogram", ptr(idx), n, top_k, num_experts, ptr(ws), ws.numel(), ptr(counts), None, s
        )
    return top_scores, idx, counts, scores


@router.register_fake
def _(logits, expert_bias, num_experts, top_k, score_func, num_expert_groups, num_limited_groups,
      route_norm, route_scale, force_load_balance, with_counts=True):
    n = logits.shape[0]
    return (
        logits.new_empty(n, top_k, dtype=torch.float32),
        logits.new_empty(n, top_k, dtype=torch.int64),
        logits.new_empty(num_experts if with_counts else 0, dtype=torch.int64),
        logits.new_empty(logits.shape, dtype=torch.float32),
    )


@torch.library.custom_op("moe_mi355x::router_backward", mutates_args=())
def router_backward(
    grad_top_scores: Tensor, scores: Tensor, selected_experts: Tensor, score_func: int,
    route_norm: bool, route_scale: float,
) -> Tensor:
    require_gpu(grad_top_scores, scores, selected_experts)
    g = grad_top_scores.float().contiguous()
    n, e = scores.shape
    k = selected_experts.shape[1]
    out = torch.empty_like(scores)
    call(
        "moe_router_bwd", ptr(g), ptr(scores), ptr(selected_experts), n, e, k, score_func,
                             int(route_norm), route_scale, ptr(out), stream_of(scores)
    )
    return out


@router_backward.register_fake
def _(grad_top_scores, scores, selected_experts, score_func, route_norm, route_scale):
    return torch.empty_like(scores)


def _router_setup(ctx, inputs, output):
    (_logits, _bias, _e, _k, score_func, _g, _gk, route_norm, route_scale, _flb, _wc) = inputs
    _top, idx, counts, scores = output
    ctx.save_for_backward(scores, idx)
    ctx.cfg = (score_func, route_norm, route_scale)
    ctx.mark_non_differentiable(idx, counts, scores)
    ctx.set_materialize_grads(False)  # no zero-filled grads for the index / saved outputs


def _router_bwd(ctx, g_top, _g_idx, _g_counts, _g_scores):
    scores, idx = ctx.saved_tensors
    score_func, route_norm, route_scale = ctx.cfg
    if g_top is None:
        g_top = torch.zeros(idx.shape, dtype=torch.float32, device=idx.device)
    grad_logits = router_backward(g_top, scores, idx, score_func, route_norm, route_scale)
    return grad_logits, None, None, None, None, None, None, None, None, None, None


router.register_autograd(_router_bwd, setup_context=_router_setup)


# ---------------------------------------------------------------------------
# the gate's backward on bf16 GEMMs: exact three-term split, dW reduction
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::gate_grad_split3", mutates_args=())
def gate_grad_split3(grad_logits: Tensor) -> Tensor:
    """fp32 [N, C] -> bf16 [N, 3C] (hi | mid | lo) with hi + mid + lo == grad_logits."""
    require_gpu(grad_logits)
    d = grad_logits.float().contiguous()
    n, c = d.shape
    out = torch.empty(n, 3 * c, dtype=torch.bfloat16, device=d.device)
    call("moe_gate_grad_split3", ptr(d), n, c, ptr(out), stream_of(d))
    return out


@gate_grad_split3.register_fake
def _(grad_logits):
    n, c = grad_logits.shape
    return grad_logits.new_empty(n, 3 * c, dtype=torch.bfloat16)


@torch.library.custom_op("moe_mi355x::gate_dw_reduce", mutates_args=())
def gate_dw_reduce(partials: Tensor, num_experts: int) -> Tensor:
    """fp32 partials [3E, D] or [2, 3E, D] (token halves) -> bf16 [E, D]:
    bf16((hi + mid) + lo) of the half sums."""
    require_gpu(partials)
    p = partials.float().contiguous()
    parts = 2 if p.dim() == 3 else 1
    d = p.shape[-1]
    if p.shape[-2] != 3 * num_experts or (parts == 2 and p.shape[0] != 2):
        raise ValueError(f"gate_dw_reduce: partials {tuple(p.shape)} for {num_experts} experts")
    out = torch.empty(num_experts, d, dtype=torch.bfloat16, device=p.device)
    call("moe_gate_dw_reduce", ptr(p), parts, num_experts, d, ptr(out), stream_of(p))
    return out


@gate_dw_reduce.register_fake
def _(partials, num_experts):
    return partials.new_empty(num_experts, partials.shape[-1], dtype=torch.bfloat16)


# ---------------------------------------------------------------------------
# shared expert SwiGLU between its GEMMs (feed_forward.py:53-54)
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::swiglu_forward", mutates_args=())
def swiglu_forward(a1: Tensor, a3: Tensor) -> Tensor:
    """h = silu(a1) * a3 with torch's roundings; a1, a3 [..., Hs] bf16 or fp32."""
    require_gpu(a1, a3)
    if a1.shape != a3.shape or a1.dtype != a3.dtype:
        raise ValueError("swiglu_forward: a1 and a3 must have one shape and dtype")
    a1c, a3c = a1.contiguous(), a3.contiguous()
    hs = a1.shape[-1]
    h = torch.empty_like(a1c)
    call("moe_swiglu_fwd", ptr(a1c), ptr(a3c), a1c.numel() // max(hs, 1), hs, _dtype_code(a1c), ptr(h),
         stream_of(a1c))
    return h


@swiglu_forward.register_fake
def _(a1, a3):
    return torch.empty_like(a1)


@torch.library.custom_op("moe_mi355x::swiglu_backward", mutates_args=())
def swiglu_backward(dh: Tensor, a1: Tensor, a3: Tensor) -> Tensor:
    """dgu [rows, 2 Hs]: silu_backward(dh * a3, a1) | dh * silu(a1), torch's roundings."""
    require_gpu(dh, a1, a3)
    if not (dh.shape == a1.shape == a3.shape) or not (dh.dtype == a1.dtype == a3.dtype):
        raise ValueError("swiglu_backward: dh, a1 and a3 must have one shape and dtype")
    hs = a1.shape[-1]
    rows = a1.numel() // max(hs, 1)
    dhc, a1c, a3c = dh.contiguous(), a1.contiguous(), a3.contiguous()
    dgu = torch.empty(rows, 2 * hs, dtype=a1.dtype, device=a1.device)
    call("moe_swiglu_bwd", ptr(dhc), ptr(a1c), ptr(a3c), rows, hs, _dtype_code(a1c), ptr(dgu), stream_of(a1c))
    return dgu


@swiglu_backward.register_fake
def _(dh, a1, a3):
    hs = a1.shape[-1]
    return a1.new_empty(a1.numel() // max(hs, 1), 2 * hs)


# ---------------------------------------------------------------------------
# reorder: counting-sort permutation by expert
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::reorder", mutates_args=())
def reorder(
    top_scores: Tensor, selected_experts: Tensor, num_experts: int
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Returns (scores_sorted [R] f32, token_idx [R] i64, counts [E] i64,
    offsets [E] i32, slot_pos [N,K] i32, tok_pos [N,K] i32)."""
    require_gpu(top_scores, selected_experts)
    idx = selected_experts.contiguous()
    ts = top_scores.float().contiguous()
    n, k = idx.shape
    dev = idx.device
    r = n * k
    scores_sorted = torch.empty(r, dtype=torch.float32, device=dev)
    token_idx = torch.empty(r, dtype=torch.int64, device=dev)
    counts = torch.empty(num_experts, dtype=torch.int64, device=dev)
    offsets = torch.empty(num_experts, dtype=torch.int32, device=dev)
    slot_pos = torch.empty(n, k, dtype=torch.int32, device=dev)
    tok_pos = torch.empty(n, k, dtype=torch.int32, device=dev)
    ws = _workspace(n, num_experts, dev)
    call(
        "moe_reorder", ptr(idx), ptr(ts), n, k, num_experts, ptr(ws), ws.numel(),
                          ptr(scores_sorted), ptr(token_idx), ptr(counts), ptr(offsets),
                          ptr(slot_pos), ptr(tok_pos), stream_of(idx)
    )
    return scores_sorted, token_idx, counts, offsets, slot_pos, tok_pos


@reorder.register_fake
def _(top_scores, selected_experts, num_experts):
    n, k = selected_experts.shape
    e = selected_experts
    return (
        e.new_empty(n * k, dtype=torch.float32),
        e.new_empty(n * k, dtype=torch.int64),
        e.new_empty(num_experts, dtype=torch.int64),
        e.new_empty(num_experts, dtype=torch.int32),
        e.new_empty(n, k, dtype=torch.int32),
        e.new_empty(n, k, dtype=torch.int32),
    )


@torch.library.custom_op("moe_mi355x::reorder_backward", mutates_args=())
def reorder_backward(grad_scores_sorted: Tensor, slot_pos: Tensor) -> Tensor:
    require_gpu(grad_scores_sorted, slot_pos)
    g = grad_scores_sorted.float().contiguous()
    n, k = slot_pos.shape
    out = torch.empty(n, k, dtype=torch.float32, device=g.device)
    call(
        "moe_reorder_bwd", ptr(g), ptr(slot_pos), n, k, ptr(out), stream_of(g)
    )
    return out


@reorder_backward.register_fake
def _(grad_scores_sorted, slot_pos):
    return slot_pos.new_empty(slot_pos.shape, dtype=torch.float32)


def _reorder_setup(ctx, inputs, output):
    _ts, _idx, _e = inputs
    _ss, token_idx, counts, offsets, slot_pos, tok_pos = output
    ctx.save_for_backward(slot_pos)
    ctx.mark_non_differentiable(token_idx, counts, offsets, slot_pos, tok_pos)
    ctx.set_materialize_grads(False)  # no zero-filled grads for the index / saved outputs


def _reorder_bwd(ctx, g_sorted, *_ignored):
    (slot_pos,) = ctx.saved_tensors
    if g_sorted is None:
        return None, None, None
    return reorder_backward(g_sorted, slot_pos), None, None


reorder.register_autograd(_reorder_bwd, setup_context=_reorder_setup)


# ---------------------------------------------------------------------------
# permute: routed_input = x[token_idx] (* score)
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::permute", mutates_args=())
def permute(x: Tensor, slot_pos: Tensor, tok_pos: Tensor, scores_sorted: Tensor | None) -> Tensor:
    require_gpu(x, slot_pos, scores_sorted)
    x = x.contiguous()
    n, d = x.shape
    k = slot_pos.shape[1]
    out = x.new_empty(n * k, d)
    sc = scores_sorted.float().contiguous() if scores_sorted is not None else None
    call(
        "moe_permute", ptr(x), ptr(slot_pos), ptr(sc), n, d, k, _dtype_code(x), ptr(out), stream_of(x)
    )
    return out


@permute.register_fake
def _(x, slot_pos, tok_pos, scores_sorted):
    return x.new_empty(x.shape[0] * slot_pos.shape[1], x.shape[1])


@torch.library.custom_op("moe_mi355x::permute_backward", mutates_args=())
def permute_backward(
    grad_routed: Tensor, x: Tensor, tok_pos: Tensor, scores_sorted: Tensor | None, round_each: bool
) -> tuple[Tensor, Tensor]:
    require_gpu(grad_routed, x, tok_pos, scores_sorted)
    g = grad_routed.contiguous()
    n, d = x.shape
    k = tok_pos.shape[1]
    grad_x = x.new_empty(n, d)
    grad_s = torch.empty(n * k if scores_sorted is not None else 0, dtype=torch.float32, device=x.device)
    sc = scores_sorted.float().contiguous() if scores_sorted is not None else None
    call(
        "moe_permute_bwd", ptr(g), ptr(x), ptr(tok_pos), ptr(sc), n, d, k, _dtype_code(x),
                              int(round_each), ptr(grad_x), ptr(grad_s) if sc is not None else None,
                              stream_of(x)
    )
    return grad_x, grad_s


@permute_backward.register_fake
def _(grad_routed, x, tok_pos, scores_sorted, round_each):
    k = tok_pos.shape[1]
    ns = x.shape[0] * k if scores_sorted is not None else 0
    return x.new_empty(x.shape), x.new_empty(ns, dtype=torch.float32)


def _permute_setup(ctx, inputs, output):
    x, slot_pos, tok_pos, scores_sorted = inputs
    ctx.has_scores = scores_sorted is not None
    ctx.save_for_backward(x, tok_pos, scores_sorted if scores_sorted is not None else None)


def _permute_bwd(ctx, g):
    x, tok_pos, scores_sorted = ctx.saved_tensors
    grad_x, grad_s = permute_backward(g, x, tok_pos, scores_sorted if ctx.has_scores else None,
                                      PERMUTE_BWD_ROUND_EACH)
    return grad_x, None, None, (grad_s if ctx.has_scores else None)


permute.register_autograd(_permute_bwd, setup_context=_permute_setup)


# ---------------------------------------------------------------------------
# grouped SwiGLU experts: _run_experts_grouped_mm
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::grouped_swiglu", mutates_args=())
def grouped_swiglu(
    x: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """bf16 grouped SwiGLU. Returns (y [R,D], g [R,H], u [R,H], h [R,H]); g, u, h are
    the saved activations for the backward."""
    require_gpu(x, w1, w2, w3, num_tokens_per_expert)
    for t, name in ((x, "x"), (w1, "w1"), (w2, "w2"), (w3, "w3")):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"grouped_swiglu expects bfloat16 {name}, got {t.dtype}")
    x, w1, w2, w3 = x.contiguous(), w1.contiguous(), w2.contiguous(), w3.contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    r, d = x.shape
    e, h_dim, _ = w1.shape
    g = x.new_empty(r, h_dim)
    u = x.new_empty(r, h_dim)
    h = x.new_empty(r, h_dim)
    y = x.new_empty(r, d)
    s = stream_of(x)
    call("moe_grouped_gemm_gate_up", ptr(x), ptr(w1), ptr(w3), ptr(counts), r, e, d, h_dim,
         ptr(g), ptr(u), ptr(h), s)
    call("moe_grouped_gemm_down", ptr(h), ptr(w2), ptr(counts), r, e, d, h_dim, ptr(y), s)
    return y, g, u, h


@grouped_swiglu.register_fake
def _(x, w1, w2, w3, num_tokens_per_expert):
    r, d = x.shape
    h_dim = w1.shape[1]
    return x.new_empty(r, d), x.new_empty(r, h_dim), x.new_empty(r, h_dim), x.new_empty(r, h_dim)


@torch.library.custom_op("moe_mi355x::grouped_swiglu_backward", mutates_args=())
def grouped_swiglu_backward(
    dy: Tensor, x: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor,
    g: Tensor, u: Tensor, h: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    require_gpu(dy, x, w1, w2, w3, num_tokens_per_expert, g, u, h)
    dy = dy.to(torch.bfloat16).contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    r, d = x.shape
    e, h_dim, _ = w1.shape
    dgu = x.new_empty(r, 2 * h_dim)
    dx = x.new_empty(r, d)
    dw1 = torch.empty_like(w1)
    dw2 = torch.empty_like(w2)
    dw3 = torch.empty_like(w3)
    s = stream_of(x)
    call("moe_grouped_gemm_bwd_dgu", ptr(dy), ptr(w2), ptr(g), ptr(u), ptr(counts), r, e, d, h_dim,
         ptr(dgu), s)
    call("moe_grouped_gemm_bwd_dx", ptr(dgu), ptr(w1), ptr(w3), ptr(counts), r, e, d, h_dim, ptr(dx), s)
    call("moe_grouped_gemm_bwd_dw13", ptr(dgu), ptr(x), ptr(counts), r, e, d, h_dim, ptr(dw1),
         ptr(dw3), s)
    call("moe_grouped_gemm_bwd_dw2", ptr(dy), ptr(h), ptr(counts), r, e, d, h_dim, ptr(dw2), s)
    return dx, dw1, dw2, dw3


@grouped_swiglu_backward.register_fake
def _(dy, x, w1, w2, w3, num_tokens_per_expert, g, u, h):
    return x.new_empty(x.shape), torch.empty_like(w1), torch.empty_like(w2), torch.empty_like(w3)


def _gs_setup(ctx, inputs, output):
    x, w1, w2, w3, counts = inputs
    _y, g, u, h = output
    ctx.save_for_backward(x, w1, w2, w3, counts, g, u, h)
    ctx.mark_non_differentiable(g, u, h)
    ctx.set_materialize_grads(False)  # no zero-filled grads for the index / saved outputs


def _gs_bwd(ctx, dy, _dg, _du, _dh):
    x, w1, w2, w3, counts, g, u, h = ctx.saved_tensors
    if dy is None:
        return None, None, None, None, None
    dx, dw1, dw2, dw3 = grouped_swiglu_backward(dy, x, w1, w2, w3, counts, g, u, h)
    return dx, dw1, dw2, dw3, None


grouped_swiglu.register_autograd(_gs_bwd, setup_context=_gs_setup)


# ---------------------------------------------------------------------------
# fp32 grouped SwiGLU experts: _run_experts_for_loop in the input dtype
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::grouped_swiglu_f32", mutates_args=())
def grouped_swiglu_f32(
    x: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """fp32 grouped SwiGLU (every product and sum in fp32, as the reference's
    fp32 per-expert matmuls, moe.py:24-50). Returns (y [R,D], g, u, h [R,H]);
    rows past sum(counts) of y are zero."""
    require_gpu(x, w1, w2, w3, num_tokens_per_expert)
    for t, name in ((x, "x"), (w1, "w1"), (w2, "w2"), (w3, "w3")):
        if t.dtype != torch.float32:
            raise TypeError(f"grouped_swiglu_f32 expects float32 {name}, got {t.dtype}")
    x, w1, w2, w3 = x.contiguous(), w1.contiguous(), w2.contiguous(), w3.contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    r, d = x.shape
    e, h_dim, _ = w1.shape
    g = x.new_zeros(r, h_dim)
    u = x.new_zeros(r, h_dim)
    h = x.new_zeros(r, h_dim)
    y = x.new_zeros(r, d)
    s = stream_of(x)
    call("moe_grouped_gemm_f32_gate_up", ptr(x), ptr(w1), ptr(w3), ptr(counts), r, e, d, h_dim,
         ptr(g), ptr(u), ptr(h), s)
    call("moe_grouped_gemm_f32_down", ptr(h), ptr(w2), ptr(counts), r, e, d, h_dim, ptr(y), s)
    return y, g, u, h


@grouped_swiglu_f32.register_fake
def _(x, w1, w2, w3, num_tokens_per_expert):
    r, d = x.shape
    h_dim = w1.shape[1]
    return x.new_empty(r, d), x.new_empty(r, h_dim), x.new_empty(r, h_dim), x.new_empty(r, h_dim)


@torch.library.custom_op("moe_mi355x::grouped_swiglu_f32_backward", mutates_args=())
def grouped_swiglu_f32_backward(
    dy: Tensor, x: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor,
    g: Tensor, u: Tensor, h: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    require_gpu(dy, x, w1, w2, w3, num_tokens_per_expert, g, u, h)
    dy = dy.to(torch.float32).contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    r, d = x.shape
    e, h_dim, _ = w1.shape
    dg = x.new_zeros(r, h_dim)
    du = x.new_zeros(r, h_dim)
    dx = x.new_zeros(r, d)
    dw1 = torch.empty_like(w1)
    dw2 = torch.empty_like(w2)
    dw3 = torch.empty_like(w3)
    s = stream_of(x)
    call("moe_grouped_gemm_f32_bwd_dgu", ptr(dy), ptr(w2), ptr(g), ptr(u), ptr(counts), r, e, d, h_dim,
         ptr(dg), ptr(du), s)
    call("moe_grouped_gemm_f32_bwd_dx", ptr(dg), ptr(du), ptr(w1), ptr(w3), ptr(counts), r, e, d, h_dim,
         ptr(dx), s)
    call("moe_grouped_gemm_f32_bwd_dw", ptr(dg), ptr(x), ptr(counts), r, e, h_dim, d, ptr(dw1), s)
    call("moe_grouped_gemm_f32_bwd_dw", ptr(du), ptr(x), ptr(counts), r, e, h_dim, d, ptr(dw3), s)
    call("moe_grouped_gemm_f32_bwd_dw", ptr(dy), ptr(h), ptr(counts), r, e, d, h_dim, ptr(dw2), s)
    return dx, dw1, dw2, dw3


@grouped_swiglu_f32_backward.register_fake
def _(dy, x, w1, w2, w3, num_tokens_per_expert, g, u, h):
    return x.new_empty(x.shape), torch.empty_like(w1), torch.empty_like(w2), torch.empty_like(w3)


def _gs32_bwd(ctx, dy, _dg, _du, _dh):
    x, w1, w2, w3, counts, g, u, h = ctx.saved_tensors
    if dy is None:
        return None, None, None, None, None
    dx, dw1, dw2, dw3 = grouped_swiglu_f32_backward(dy, x, w1, w2, w3, counts, g, u, h)
    return dx, dw1, dw2, dw3, None


grouped_swiglu_f32.register_autograd(_gs32_bwd, setup_context=_gs_setup)


# ---------------------------------------------------------------------------
# combine: out = shared + sum of a token's routed rows (deterministic)
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::combine", mutates_args=())
def combine(
    shared_out: Tensor | None, routed_output: Tensor, slot_pos: Tensor, tok_pos: Tensor,
    scores_sorted: Tensor | None,
) -> Tensor:
    require_gpu(shared_out, routed_output, tok_pos, scores_sorted)
    routed = routed_output.contiguous()
    n, k = tok_pos.shape
    d = routed.shape[1]
    base = shared_out.to(routed.dtype).contiguous() if shared_out is not None else None
    out = routed.new_empty(n, d)
    sc = scores_sorted.float().contiguous() if scores_sorted is not None else None
    call(
        "moe_combine", ptr(base), ptr(routed), ptr(tok_pos), ptr(sc), n, d, k, _dtype_code(routed),
                          ptr(out), stream_of(routed)
    )
    return out


@combine.register_fake
def _(shared_out, routed_output, slot_pos, tok_pos, scores_sorted):
    return routed_output.new_empty(tok_pos.shape[0], routed_output.shape[1])


@torch.library.custom_op("moe_mi355x::combine_backward", mutates_args=())
def combine_backward(
    grad_out: Tensor, routed_output: Tensor, slot_pos: Tensor, tok_pos: Tensor,
    scores_sorted: Tensor | None,
) -> tuple[Tensor, Tensor]:
    require_gpu(grad_out, routed_output, slot_pos, tok_pos, scores_sorted)
    g = grad_out.to(routed_output.dtype).contiguous()
    n, k = tok_pos.shape
    d = g.shape[1]
    grad_routed = g.new_empty(n * k, d)
    grad_s = torch.empty(n * k if scores_sorted is not None else 0, dtype=torch.float32, device=g.device)
    sc = scores_sorted.float().contiguous() if scores_sorted is not None else None
    call(
        "moe_combine_bwd", ptr(g), ptr(routed_output), ptr(slot_pos), ptr(tok_pos), ptr(sc), n, d, k,
                              _dtype_code(g), ptr(grad_routed), ptr(grad_s) if sc is not None else None,
                              stream_of(g)
    )
    return grad_routed, grad_s


@combine_backward.register_fake
def _(grad_out, routed_output, slot_pos, tok_pos, scores_sorted):
    n, k = tok_pos.shape
    ns = n * k if scores_sorted is not None else 0
    return routed_output.new_empty(n * k, routed_output.shape[1]), grad_out.new_empty(ns, dtype=torch.float32)


def _combine_setup(ctx, inputs, output):
    shared_out, routed_output, slot_pos, tok_pos, scores_sorted = inputs
    ctx.has_shared = shared_out is not None
    ctx.shared_dtype = shared_out.dtype if shared_out is not None else None
    ctx.has_scores = scores_sorted is not None
    ctx.save_for_backward(routed_output if ctx.has_scores else None, slot_pos, tok_pos, scores_sorted)


def _combine_bwd(ctx, g):
    routed, slot_pos, tok_pos, scores_sorted = ctx.saved_tensors
    if ctx.has_scores:
        grad_routed, grad_s = combine_backward(g, routed, slot_pos, tok_pos, scores_sorted)
    else:
        dummy = g.new_empty(0, g.shape[1])
        grad_routed, _ = combine_backward(g, dummy, slot_pos, tok_pos, None)
        grad_s = None
    grad_shared = g.to(ctx.shared_dtype) if ctx.has_shared else None
    return grad_shared, grad_routed, None, None, grad_s


combine.register_autograd(_combine_bwd, setup_context=_combine_setup)


# ---------------------------------------------------------------------------
# gpt-oss experts: biased, clamped SwiGLU with interleaved mlp1 rows
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::grouped_swiglu_oss", mutates_args=())
def grouped_swiglu_oss(
    x: Tensor, mlp1_weight: Tensor, mlp1_bias: Tensor, mlp2_weight: Tensor, mlp2_bias: Tensor,
    num_tokens_per_expert: Tensor, swiglu_limit: float,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """gpt-oss grouped experts (gpt_oss/moe.py:92-122) in bf16: returns y [R, D]
    and the saved g, u (biased pre-clamp halves of h1) and h [R, H]."""
    require_gpu(x, mlp1_weight, mlp1_bias, mlp2_weight, mlp2_bias, num_tokens_per_expert)
    x, w1, w2 = (t.contiguous() for t in (x, mlp1_weight, mlp2_weight))
    for t, name in ((x, "x"), (w1, "mlp1_weight"), (w2, "mlp2_weight")):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"grouped_swiglu_oss expects bfloat16 {name}, got {t.dtype}")
    b1 = mlp1_bias.to(torch.bfloat16).contiguous()
    b2 = mlp2_bias.to(torch.bfloat16).contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    r, d = x.shape
    e, h2, _ = w1.shape
    h_dim = h2 // 2
    s = stream_of(x)
    g = x.new_empty(r, h_dim)
    u = x.new_empty(r, h_dim)
    h = x.new_empty(r, h_dim)
    y = x.new_empty(r, d)
    call("moe_grouped_gemm_oss_gate_up", ptr(x), ptr(w1), ptr(b1), ptr(counts), r, e, d, h_dim, float(swiglu_limit),
         ptr(g), ptr(u), ptr(h), s)
    call("moe_grouped_gemm_oss_down", ptr(h), ptr(w2), ptr(b2), ptr(counts), r, e, d, h_dim, ptr(y), s)
    return y, g, u, h


@grouped_swiglu_oss.register_fake
def _(x, mlp1_weight, mlp1_bias, mlp2_weight, mlp2_bias, num_tokens_per_expert, swiglu_limit):
    r, d = x.shape
    h_dim = mlp1_weight.shape[1] // 2
    return x.new_empty(r, d), x.new_empty(r, h_dim), x.new_empty(r, h_dim), x.new_empty(r, h_dim)


@torch.library.custom_op("moe_mi355x::grouped_swiglu_oss_backward", mutates_args=())
def grouped_swiglu_oss_backward(
    dy: Tensor, x: Tensor, mlp1_weight: Tensor, mlp1_bias: Tensor, mlp2_weight: Tensor, mlp2_bias: Tensor,
    num_tokens_per_expert: Tensor, g: Tensor, u: Tensor, h: Tensor, swiglu_limit: float,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients (dx, dmlp1_weight, dmlp1_bias, dmlp2_weight, dmlp2_bias); the
    bias gradients are fp32 per-expert sums in a fixed order, cast to the bias dtype."""
    require_gpu(dy, x, mlp1_weight, mlp2_weight, num_tokens_per_expert, g, u, h)
    dy = dy.to(torch.bfloat16).contiguous()
    x, w1, w2 = (t.contiguous() for t in (x, mlp1_weight, mlp2_weight))
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    r, d = x.shape
    e, h2, _ = w1.shape
    h_dim = h2 // 2
    s = stream_of(x)
    dgu = x.new_empty(r, 2 * h_dim)
    call("moe_grouped_gemm_oss_bwd_dgu", ptr(dy), ptr(w2), ptr(g), ptr(u), ptr(counts), r, e, d, h_dim,
         float(swiglu_limit), ptr(dgu), s)
    dx = x.new_empty(r, d)
    call("moe_grouped_gemm_oss_bwd_dx", ptr(dgu), ptr(w1), ptr(counts), r, e, d, h_dim, ptr(dx), s)
    dw1 = torch.empty_like(w1)
    call("moe_grouped_gemm_oss_bwd_dw1", ptr(dgu), ptr(x), ptr(counts), r, e, d, h_dim, ptr(dw1), s)
    dw2 = torch.empty_like(w2)
    call("moe_grouped_gemm_bwd_dw2", ptr(dy), ptr(h), ptr(counts), r, e, d, h_dim, ptr(dw2), s)
    db1 = torch.empty(e, 2 * h_dim, dtype=torch.float32, device=x.device)
    call("moe_grouped_col_sum", ptr(dgu), 2 * h_dim, ptr(counts), r, e, h_dim, ptr(db1), 2 * h_dim, 2, s)
    call("moe_grouped_col_sum", dgu.data_ptr() + 2 * h_dim, 2 * h_dim, ptr(counts), r, e, h_dim,
         db1.data_ptr() + 4, 2 * h_dim, 2, s)
    db2 = torch.empty(e, d, dtype=torch.float32, device=x.device)
    call("moe_grouped_col_sum", ptr(dy), d, ptr(counts), r, e, d, ptr(db2), d, 1, s)
    return dx, dw1, db1.to(mlp1_bias.dtype), dw2, db2.to(mlp2_bias.dtype)


@grouped_swiglu_oss_backward.register_fake
def _(dy, x, mlp1_weight, mlp1_bias, mlp2_weight, mlp2_bias, num_tokens_per_expert, g, u, h, swiglu_limit):
    return (x.new_empty(x.shape), torch.empty_like(mlp1_weight), torch.empty_like(mlp1_bias),
            torch.empty_like(mlp2_weight), torch.empty_like(mlp2_bias))


def _oss_setup(ctx, inputs, output):
    x, w1, b1, w2, b2, counts, limit = inputs
    _, g, u, h = output
    ctx.save_for_backward(x, w1, b1, w2, b2, counts, g, u, h)
    ctx.swiglu_limit = limit
    ctx.set_materialize_grads(False)


def _oss_bwd(ctx, dy, _dg, _du, _dh):
    x, w1, b1, w2, b2, counts, g, u, h = ctx.saved_tensors
    if dy is None:
        return None, None, None, None, None, None, None
    dx, dw1, db1, dw2, db2 = grouped_swiglu_oss_backward(dy, x, w1, b1, w2, b2, counts, g, u, h, ctx.swiglu_limit)
    return dx, dw1, db1, dw2, db2, None, None


grouped_swiglu_oss.register_autograd(_oss_bwd, setup_context=_oss_setup)


# ---------------------------------------------------------------------------
# fp8 e4m3 grouped SwiGLU experts (dynamic rowwise scaling, fp32 accumulate)
# ---------------------------------------------------------------------------
FP8 = torch.uint8  # fp8 e4m3fn bytes as produced by the quantizers


def _quant_rows(x: Tensor, cols: int) -> tuple[Tensor, Tensor]:
    """x viewed as [rows, cols] bf16 -> (q uint8 [rows, cols], scale f32 [rows])."""
    rows = x.numel() // cols
    q = torch.empty(rows, cols, dtype=FP8, device=x.device)
    s = torch.empty(rows, dtype=torch.float32, device=x.device)
    call("moe_fp8_quant_rows", ptr(x), rows, cols, ptr(q), ptr(s), stream_of(x))
    return q, s


# widest rows the row quantizers with a column amax on the side take (their
# rows stay in registers)
AMAX_SIDE_MAX_COLS = 8192


def _amax_shape(e: int, cols: int) -> tuple[int, ...]:
    """Shape of a column amax taken on the side of a row quantization: [E, cols],
    or empty when the rows are too wide (the transposed quantizer then takes its
    own amax pass)."""
    return (e, cols) if cols <= AMAX_SIDE_MAX_COLS else (0,)


def _quant_rows_colamax(w: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """w [E, A, B] bf16 -> (q [E, A, B] fp8 with a scale per row, scale [E * A],
    column amax [E, B] over A): the row quantization and, on the side, what the
    transposed one needs, from one read."""
    e, a, b = w.shape
    if b > AMAX_SIDE_MAX_COLS:
        q, s = _quant_rows(w, b)
        return q.view(e, a, b), s, w.new_empty(0, dtype=torch.float32)
    q = torch.empty(e, a, b, dtype=FP8, device=w.device)
    s = torch.empty(e * a, dtype=torch.float32, device=w.device)
    amax = torch.zeros(e, b, dtype=torch.float32, device=w.device)
    call("moe_fp8_quant_rows_colamax", ptr(w), e, a, b, ptr(q), ptr(s), ptr(amax), stream_of(w))
    return q, s, amax


def _quant_rows_groupamax(x: Tensor, counts: Tensor, e: int, pieces: int = 1) -> tuple[Tensor, Tensor, Tensor]:
    """x [R, C] bf16 in expert token groups -> (q [R, C] fp8 with a scale per row
    piece of C / pieces columns, scale [R * pieces], the column amax [E, C] of
    each group): the row quantization and, on the side, what the token-transposed
    one needs, from one read."""
    r, c = x.shape
    if c > AMAX_SIDE_MAX_COLS:
        q, sc = _quant_rows(x, c // pieces)
        return q.view(r, c), sc, x.new_empty(0, dtype=torch.float32)
    q = torch.empty(r, c, dtype=FP8, device=x.device)
    sc = torch.empty(r * pieces, dtype=torch.float32, device=x.device)
    amax = torch.zeros(e, c, dtype=torch.float32, device=x.device)
    call("moe_fp8_quant_rows_groupamax", ptr(x), ptr(counts), r, e, c, pieces, ptr(q), ptr(sc), ptr(amax),
         stream_of(x))
    return q, sc, amax


def _quant_cols_t(w: Tensor, amax: Tensor, q: Tensor, q_offset: int, q_estride: int, q_ld: int, scale: Tensor,
                  s_offset: int, s_estride: int) -> None:
    """Per expert and column of w [E, A, B]: the scale of the column amax and the
    column quantized as a row of q (transposed); from the known amax when there
    is one (one read of w), else with its own amax pass."""
    e, a, b = w.shape
    qp, sp = q.data_ptr() + q_offset, scale.data_ptr() + 4 * s_offset
    if amax.numel():
        call("moe_fp8_quant_cols_t_amax", ptr(w), ptr(amax), e, a, b, qp, q_estride, q_ld, sp, s_estride,
             stream_of(w))
    else:
        call("moe_fp8_quant_cols_t", ptr(w), e, a, b, qp, q_estride, q_ld, sp, s_estride, stream_of(w))


def _padded_rows(r: int, e: int) -> int:
    """Width of the token-transposed layout (token groups 128-aligned): a multiple
    of 128, so that every row and every group in it starts on a 128-byte line."""
    n = lib().moe_fp8_padded_rows(r, e)
    return (n + 127) // 128 * 128


def _quant_tokens_t(x: Tensor, counts: Tensor, e: int, rpad: int,
                    amax: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """x [R, C] bf16 in expert token groups -> (q [C, rpad], scale [E, C]); from
    the groups' known column amax when there is one (one read of x), else with
    its own amax pass."""
    r, c = x.shape
    q = torch.empty(c, rpad, dtype=FP8, device=x.device)
    s = torch.empty(e, c, dtype=torch.float32, device=x.device)
    if amax is not None and amax.numel():
        call("moe_fp8_quant_tokens_t_amax", ptr(x), ptr(amax), ptr(counts), r, e, c, rpad, ptr(q), ptr(s),
             stream_of(x))
    else:
        call("moe_fp8_quant_tokens_t", ptr(x), ptr(counts), r, e, c, rpad, ptr(q), ptr(s), stream_of(x))
    return q, s


@torch.library.custom_op("moe_mi355x::grouped_swiglu_fp8", mutates_args=())
def grouped_swiglu_fp8(
    x: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """fp8 e4m3 grouped SwiGLU: x, h quantized per token row, weights per
    output row; fp32 accumulate; bf16 outputs (y, g, u, h), then the column
    amax the backward's transposed quantizations use, taken on the side of the
    forward's: the weights' over their output rows (w1, w3 [E, D], w2 [E, H])
    and x's and h's over each expert's tokens ([E, D], [E, H])."""
    require_gpu(x, w1, w2, w3, num_tokens_per_expert)
    for t, name in ((x, "x"), (w1, "w1"), (w2, "w2"), (w3, "w3")):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"grouped_swiglu_fp8 expects bfloat16 {name}, got {t.dtype}")
    x, w1, w2, w3 = x.contiguous(), w1.contiguous(), w2.contiguous(), w3.contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    qx, sx, amx = _quant_rows_groupamax(x, counts, w1.shape[0])
    y, g, u, h, am1, am3, am2, amh = _fp8_experts_forward(qx, sx, w1, w2, w3, counts)
    return y, g, u, h, am1, am3, am2, amx, amh


def _fp8_experts_forward(qx: Tensor, sx: Tensor, w1: Tensor, w2: Tensor, w3: Tensor,
                         counts: Tensor) -> tuple[Tensor, ...]:
    """grouped_swiglu_fp8 from the row-quantized routed rows (qx, sx): the weights'
    quantizations, gate_up, h's quantization, down. Returns (y, g, u, h, amax_w1,
    amax_w3, amax_w2, amax_h)."""
    r, d = qx.shape
    e, h_dim, _ = w1.shape
    s = stream_of(w1)
    qw1, sw1, am1 = _quant_rows_colamax(w1)
    qw3, sw3, am3 = _quant_rows_colamax(w3)
    qw2, sw2, am2 = _quant_rows_colamax(w2)
    g = w1.new_empty(r, h_dim)
    u = w1.new_empty(r, h_dim)
    h = w1.new_empty(r, h_dim)
    y = w1.new_empty(r, d)
    call("moe_fp8_gemm_gate_up", ptr(qx), ptr(sx), ptr(qw1), ptr(sw1), ptr(qw3), ptr(sw3), ptr(counts), r, e, d,
         h_dim, ptr(g), ptr(u), ptr(h), s)
    qh, sh, amh = _quant_rows_groupamax(h, counts, e)
    call("moe_fp8_gemm_down", ptr(qh), ptr(sh), ptr(qw2), ptr(sw2), ptr(counts), r, e, d, h_dim, ptr(y), s)
    return y, g, u, h, am1, am3, am2, amh


@grouped_swiglu_fp8.register_fake
def _(x, w1, w2, w3, num_tokens_per_expert):
    r, d = x.shape
    e, h_dim = w1.shape[0], w1.shape[1]
    f32 = lambda *shape: x.new_empty(*shape, dtype=torch.float32)  # noqa: E731
    return (x.new_empty(r, d), x.new_empty(r, h_dim), x.new_empty(r, h_dim), x.new_empty(r, h_dim),
            f32(*_amax_shape(e, d)), f32(*_amax_shape(e, d)), f32(*_amax_shape(e, h_dim)),
            f32(*_amax_shape(e, d)), f32(*_amax_shape(e, h_dim)))


@torch.library.custom_op("moe_mi355x::grouped_swiglu_fp8_backward", mutates_args=())
def grouped_swiglu_fp8_backward(
    dy: Tensor, x: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor,
    g: Tensor, u: Tensor, h: Tensor, amax_w1: Tensor, amax_w3: Tensor, amax_w2: Tensor, amax_x: Tensor,
    amax_h: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Gradients of grouped_swiglu_fp8. amax_* are the forward's column amax of
    the weights and of x and h per token group (empty tensors: the transposed
    quantizers take their own)."""
    require_gpu(dy, x, w1, w2, w3, num_tokens_per_expert, g, u, h)
    dy = dy.to(torch.bfloat16).contiguous()
    x = x.contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    e = w1.shape[0]
    qdy, sdy, amdy = _quant_rows_groupamax(dy, counts, e)
    return _fp8_experts_backward(
        qdy, sdy, w1, w2, w3, counts, g, u, h, amax_w1, amax_w3, amax_w2, amax_h,
        lambda rpad: _quant_tokens_t(x, counts, e, rpad, amax_x),
        lambda rpad: _quant_tokens_t(dy, counts, e, rpad, amdy))


def _fp8_experts_backward(qdy: Tensor, sdy: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, counts: Tensor, g: Tensor,
                          u: Tensor, h: Tensor, amax_w1: Tensor, amax_w3: Tensor, amax_w2: Tensor, amax_h: Tensor,
                          x_tokens_t, dy_tokens_t) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """grouped_swiglu_fp8_backward from the row-quantized output gradient (qdy,
    sdy); x_tokens_t(rpad) and dy_tokens_t(rpad) give the token-transposed layouts
    of the routed x and dy. Returns (dx, dw1, dw2, dw3)."""
    r, d = qdy.shape
    e, h_dim, _ = w1.shape
    dev = w1.device
    s = stream_of(w1)
    # dh = dy . w2 (contraction over D): dy per row, w2 per (e, h) column over D
    qw2t = torch.empty(e, h_dim, d, dtype=FP8, device=dev)
    sw2t = torch.empty(e, h_dim, dtype=torch.float32, device=dev)
    _quant_cols_t(w2.contiguous(), amax_w2.contiguous(), qw2t, 0, h_dim * d, d, sw2t, 0, h_dim)
    dgu = w1.new_empty(r, 2 * h_dim)
    call("moe_fp8_gemm_bwd_dgu", ptr(qdy), ptr(sdy), ptr(qw2t), ptr(sw2t), ptr(g), ptr(u), ptr(counts), r, e, d,
         h_dim, ptr(dgu), s)
    # dx = dg . w1 + du . w3 (contraction over H): one scale per dg / du row half,
    # w1 and w3 per (e, d) column over H, written side by side as [E, D, 2H]
    qdgu, sdgu, amdgu = _quant_rows_groupamax(dgu, counts, e, pieces=2)
    qw13t = torch.empty(e, d, 2 * h_dim, dtype=FP8, device=dev)
    sw13t = torch.empty(e, 2, d, dtype=torch.float32, device=dev)
    _quant_cols_t(w1.contiguous(), amax_w1.contiguous(), qw13t, 0, d * 2 * h_dim, 2 * h_dim, sw13t, 0, 2 * d)
    _quant_cols_t(w3.contiguous(), amax_w3.contiguous(), qw13t, h_dim, d * 2 * h_dim, 2 * h_dim, sw13t, d, 2 * d)
    dx = w1.new_empty(r, d)
    call("moe_fp8_gemm_bwd_dx", ptr(qdgu), ptr(sdgu), ptr(qw13t), ptr(sw13t), ptr(counts), r, e, d, h_dim,
         ptr(dx), s)
    # weight gradients: contraction over each expert's tokens (per-group scales)
    rpad = _padded_rows(r, e)
    qdgut, sdgut = _quant_tokens_t(dgu, counts, e, rpad, amdgu)
    qxt, sxt = x_tokens_t(rpad)
    dw1 = torch.empty_like(w1)
    dw3 = torch.empty_like(w3)
    call("moe_fp8_gemm_bwd_dw13", ptr(qdgut), ptr(sdgut), ptr(qxt), ptr(sxt), ptr(counts), r, rpad, e, d, h_dim,
         ptr(dw1), ptr(dw3), s)
    qdyt, sdyt = dy_tokens_t(rpad)
    qht, sht = _quant_tokens_t(h, counts, e, rpad, amax_h)
    dw2 = torch.empty_like(w2)
    call("moe_fp8_gemm_bwd_dw2", ptr(qdyt), ptr(sdyt), ptr(qht), ptr(sht), ptr(counts), r, rpad, e, d, h_dim,
         ptr(dw2), s)
    return dx, dw1, dw2, dw3


@grouped_swiglu_fp8_backward.register_fake
def _(dy, x, w1, w2, w3, num_tokens_per_expert, g, u, h, amax_w1, amax_w3, amax_w2, amax_x, amax_h):
    return x.new_empty(x.shape), torch.empty_like(w1), torch.empty_like(w2), torch.empty_like(w3)


def _gs8_setup(ctx, inputs, output):
    x, w1, w2, w3, counts = inputs
    _y, g, u, h, *amax = output
    ctx.save_for_backward(x, w1, w2, w3, counts, g, u, h, *amax)
    ctx.mark_non_differentiable(g, u, h, *amax)
    ctx.set_materialize_grads(False)


def _gs8_bwd(ctx, dy, *_unused):
    x, w1, w2, w3, counts, g, u, h, *amax = ctx.saved_tensors
    if dy is None:
        return None, None, None, None, None
    dx, dw1, dw2, dw3 = grouped_swiglu_fp8_backward(dy, x, w1, w2, w3, counts, g, u, h, *amax)
    return dx, dw1, dw2, dw3, None


grouped_swiglu_fp8.register_autograd(_gs8_bwd, setup_context=_gs8_setup)


# ---------------------------------------------------------------------------
# MXFP8 grouped SwiGLU experts (e8m0 scales per 32 elements along the
# contraction, RCEIL; fp32 accumulate)
# ---------------------------------------------------------------------------
MX_BLOCK = 32


def _mx_quant_rows(x: Tensor, cols: int) -> tuple[Tensor, Tensor]:
    """x viewed as [rows, cols] bf16 -> (q uint8 [rows, cols], e8m0 uint8 [rows, cols / 32])."""
    rows = x.numel() // cols
    q = torch.empty(rows, cols, dtype=FP8, device=x.device)
    s = torch.empty(rows, cols // MX_BLOCK, dtype=torch.uint8, device=x.device)
    call("moe_mxfp8_quant_rows", ptr(x), rows, cols, ptr(q), ptr(s), stream_of(x))
    return q, s


def _mx_padded_rows(r: int, e: int) -> int:
    """As _padded_rows: r + 127 e rounded up to 128 (token groups 128-aligned)."""
    return (int(lib().moe_mxfp8_padded_rows(r, e)) + 127) // 128 * 128


def _mx_quant_tokens_t(x: Tensor, counts: Tensor, e: int, rpad: int) -> tuple[Tensor, Tensor]:
    """x [R, C] bf16 in expert token groups -> (q [C, rpad], e8m0 [rpad / 32, C])."""
    r, c = x.shape
    q = torch.empty(c, rpad, dtype=FP8, device=x.device)
    s = torch.empty(rpad // MX_BLOCK, c, dtype=torch.uint8, device=x.device)
    call("moe_mxfp8_quant_tokens_t", ptr(x), ptr(counts), r, e, c, rpad, ptr(q), ptr(s), stream_of(x))
    return q, s


def _check_bf16(op: str, **tensors: Tensor) -> None:
    for name, t in tensors.items():
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{op} expects bfloat16 {name}, got {t.dtype}")


def _mx_dual_tokens(x: Tensor, counts: Tensor, e: int, rpad: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """One read of x [R, C] (token groups) -> the row-wise MX layout (q [R, C],
    e8m0 [R, C / 32]) and the token-transposed one (q [C, rpad], e8m0 [rpad / 32, C])."""
    r, c = x.shape
    qr = torch.empty(r, c, dtype=FP8, device=x.device)
    sr = torch.empty(r, c // MX_BLOCK, dtype=torch.uint8, device=x.device)
    qt = torch.empty(c, rpad, dtype=FP8, device=x.device)
    st = torch.empty(rpad // MX_BLOCK, c, dtype=torch.uint8, device=x.device)
    call("moe_mxfp8_quant_dual_tokens", ptr(x), ptr(counts), r, e, c, rpad, ptr(qr), ptr(sr), ptr(qt), ptr(st),
         stream_of(x))
    return qr, sr, qt, st


def _mx_weights(w1: Tensor, w2: Tensor, w3: Tensor, transposed: bool) -> tuple[Tensor, ...]:
    """Row-wise MX layouts of w1, w3 (blocks along D) and w2 (along H); with
    `transposed`, the same reads also write the backward's layouts: w2^T
    [E, H, D] (blocks along D) and [w1^T | w3^T] [E, D, 2H] (blocks along H)."""
    e, h_dim, d = w1.shape
    dev = w1.device
    s = stream_of(w1)
    if not transposed:
        qw1, sw1 = _mx_quant_rows(w1, d)
        qw3, sw3 = _mx_quant_rows(w3, d)
        qw2, sw2 = _mx_quant_rows(w2, h_dim)
        return qw1, sw1, qw3, sw3, qw2, sw2
    qw1 = torch.empty(e * h_dim, d, dtype=FP8, device=dev)
    sw1 = torch.empty(e * h_dim, d // MX_BLOCK, dtype=torch.uint8, device=dev)
    qw3, sw3 = torch.empty_like(qw1), torch.empty_like(sw1)
    qw2 = torch.empty(e * d, h_dim, dtype=FP8, device=dev)
    sw2 = torch.empty(e * d, h_dim // MX_BLOCK, dtype=torch.uint8, device=dev)
    qw2t = torch.empty(e, h_dim, d, dtype=FP8, device=dev)
    sw2t = torch.empty(e, h_dim, d // MX_BLOCK, dtype=torch.uint8, device=dev)
    nb = 2 * h_dim // MX_BLOCK
    qw13t = torch.empty(e, d, 2 * h_dim, dtype=FP8, device=dev)
    sw13t = torch.empty(e, d, nb, dtype=torch.uint8, device=dev)
    call("moe_mxfp8_quant_dual_cols", ptr(w2), e, d, h_dim, ptr(qw2), ptr(sw2), ptr(qw2t), h_dim * d, d, ptr(sw2t),
         h_dim * (d // MX_BLOCK), d // MX_BLOCK, s)
    call("moe_mxfp8_quant_dual_cols", ptr(w1), e, h_dim, d, ptr(qw1), ptr(sw1), ptr(qw13t), d * 2 * h_dim, 2 * h_dim,
         ptr(sw13t), d * nb, nb, s)
    call("moe_mxfp8_quant_dual_cols", ptr(w3), e, h_dim, d, ptr(qw3), ptr(sw3), qw13t.data_ptr() + h_dim,
         d * 2 * h_dim, 2 * h_dim, sw13t.data_ptr() + h_dim // MX_BLOCK, d * nb, nb, s)
    return qw1, sw1, qw3, sw3, qw2, sw2, qw2t, sw2t, qw13t, sw13t


@torch.library.custom_op("moe_mi355x::grouped_swiglu_mxfp8", mutates_args=())
def grouped_swiglu_mxfp8(
    x: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor, for_backward: bool = False
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """MXFP8 grouped SwiGLU: x, h and the weights quantized in 32-element
    blocks along each GEMM's contraction; bf16 outputs (y, g, u, h). With
    `for_backward`, the same quantizer reads also produce the layouts the
    backward contracts over (x^T, h^T per token group; w1^T, w3^T, w2^T),
    returned after (y, g, u, h); otherwise those are empty."""
    require_gpu(x, w1, w2, w3, num_tokens_per_expert)
    _check_bf16("grouped_swiglu_mxfp8", x=x, w1=w1, w2=w2, w3=w3)
    x, w1, w2, w3 = x.contiguous(), w1.contiguous(), w2.contiguous(), w3.contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    r, d = x.shape
    e, h_dim, _ = w1.shape
    s = stream_of(x)
    def empty():  # distinct placeholders: custom-op outputs may not alias each other
        return x.new_empty(0, dtype=torch.uint8)
    if for_backward:
        rpad = _mx_padded_rows(r, e)
        qx, sx, qxt, sxt = _mx_dual_tokens(x, counts, e, rpad)
        qw1, sw1, qw3, sw3, qw2, sw2, qw2t, sw2t, qw13t, sw13t = _mx_weights(w1, w2, w3, True)
    else:
        qx, sx = _mx_quant_rows(x, d)
        qw1, sw1, qw3, sw3, qw2, sw2 = _mx_weights(w1, w2, w3, False)
        qxt, sxt, qw2t, sw2t, qw13t, sw13t = (empty() for _ in range(6))
    g = x.new_empty(r, h_dim)
    u = x.new_empty(r, h_dim)
    h = x.new_empty(r, h_dim)
    y = x.new_empty(r, d)
    call("moe_mxfp8_gemm_gate_up", ptr(qx), ptr(sx), ptr(qw1), ptr(sw1), ptr(qw3), ptr(sw3), ptr(counts), r, e, d,
         h_dim, ptr(g), ptr(u), ptr(h), s)
    if for_backward:
        qh, sh, qht, sht = _mx_dual_tokens(h, counts, e, rpad)
    else:
        qh, sh = _mx_quant_rows(h, h_dim)
        qht, sht = empty(), empty()
    call("moe_mxfp8_gemm_down", ptr(qh), ptr(sh), ptr(qw2), ptr(sw2), ptr(counts), r, e, d, h_dim, ptr(y), s)
    return y, g, u, h, qxt, sxt, qht, sht, qw2t, sw2t, qw13t, sw13t


@grouped_swiglu_mxfp8.register_fake
def _(x, w1, w2, w3, num_tokens_per_expert, for_backward=False):
    r, d = x.shape
    e, h_dim, _ = w1.shape
    bf = (x.new_empty(r, d), x.new_empty(r, h_dim), x.new_empty(r, h_dim), x.new_empty(r, h_dim))
    u8 = lambda *shape: x.new_empty(*shape, dtype=torch.uint8)  # noqa: E731
    if not for_backward:
        return (*bf, *(u8(0) for _ in range(8)))
    rpad = (r + e * 127 + 127) // 128 * 128  # _mx_padded_rows
    return (*bf, u8(d, rpad), u8(rpad // 32, d), u8(h_dim, rpad), u8(rpad // 32, h_dim),
            u8(e, h_dim, d), u8(e, h_dim, d // 32), u8(e, d, 2 * h_dim), u8(e, d, 2 * h_dim // 32))


@torch.library.custom_op("moe_mi355x::grouped_swiglu_mxfp8_backward", mutates_args=())
def grouped_swiglu_mxfp8_backward(
    dy: Tensor, x: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor,
    g: Tensor, u: Tensor, h: Tensor, qxt: Tensor, sxt: Tensor, qht: Tensor, sht: Tensor,
    qw2t: Tensor, sw2t: Tensor, qw13t: Tensor, sw13t: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Gradients from the forward's transposed quantizations; dy and dgu are
    quantized once each, in both layouts."""
    require_gpu(dy, x, w1, w2, w3, num_tokens_per_expert, g, u, h)
    dy = dy.to(torch.bfloat16).contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    r, d = x.shape
    e, h_dim, _ = w1.shape
    s = stream_of(x)
    rpad = _mx_padded_rows(r, e)
    if qxt.numel() == 0:  # the forward ran without for_backward
        qxt, sxt = _mx_quant_tokens_t(x.contiguous(), counts, e, rpad)
        qht, sht = _mx_quant_tokens_t(h, counts, e, rpad)
        *_, qw2t, sw2t, qw13t, sw13t = _mx_weights(w1.contiguous(), w2.contiguous(), w3.contiguous(), True)
    # dh = dy . w2 (contraction over D)
    qdy = _mx_dual_tokens(dy, counts, e, rpad)
    return _mx_experts_backward(qdy, r, d, w1, w2, w3, counts, g, u, h, qxt, sxt, qht, sht, qw2t, sw2t, qw13t,
                                sw13t, rpad)


def _mx_experts_backward(qdy, r, d, w1, w2, w3, counts, g, u, h, qxt, sxt, qht, sht, qw2t, sw2t, qw13t, sw13t, rpad):
    """dx (routed rows), dw1, dw2, dw3 of the MXFP8 experts from dy's two MX
    layouts (qdy = (q rows, e8m0 rows, q tokens^T, e8m0 tokens^T))."""
    qdy, sdy, qdyt, sdyt = qdy
    e, h_dim, _ = w1.shape
    s = stream_of(g)
    dgu = g.new_empty(r, 2 * h_dim)
    call("moe_mxfp8_gemm_bwd_dgu", ptr(qdy), ptr(sdy), ptr(qw2t), ptr(sw2t), ptr(g), ptr(u), ptr(counts), r, e, d,
         h_dim, ptr(dgu), s)
    # dx = dg . w1 + du . w3 (contraction over H; blocks never straddle the halves)
    qdgu, sdgu, qdgut, sdgut = _mx_dual_tokens(dgu, counts, e, rpad)
    dx = g.new_empty(r, d)
    call("moe_mxfp8_gemm_bwd_dx", ptr(qdgu), ptr(sdgu), ptr(qw13t), ptr(sw13t), ptr(counts), r, e, d, h_dim,
         ptr(dx), s)
    # weight gradients: contraction over each expert's tokens (groups padded to 32)
    dw1 = torch.empty_like(w1)
    dw3 = torch.empty_like(w3)
    call("moe_mxfp8_gemm_bwd_dw13", ptr(qdgut), ptr(sdgut), ptr(qxt), ptr(sxt), ptr(counts), r, rpad, e, d, h_dim,
         ptr(dw1), ptr(dw3), s)
    dw2 = torch.empty_like(w2)
    call("moe_mxfp8_gemm_bwd_dw2", ptr(qdyt), ptr(sdyt), ptr(qht), ptr(sht), ptr(counts), r, rpad, e, d, h_dim,
         ptr(dw2), s)
    return dx, dw1, dw2, dw3


@grouped_swiglu_mxfp8_backward.register_fake
def _(dy, x, w1, w2, w3, num_tokens_per_expert, g, u, h, *quantized):
    return x.new_empty(x.shape), torch.empty_like(w1), torch.empty_like(w2), torch.empty_like(w3)


def _gsmx_setup(ctx, inputs, output):
    x, w1, w2, w3, counts, _for_backward = inputs
    _y, g, u, h, *quantized = output
    ctx.save_for_backward(x, w1, w2, w3, counts, g, u, h, *quantized)
    ctx.mark_non_differentiable(g, u, h, *quantized)
    ctx.set_materialize_grads(False)


def _gsmx_bwd(ctx, dy, *_unused):
    x, w1, w2, w3, counts, g, u, h, *quantized = ctx.saved_tensors
    if dy is None:
        return None, None, None, None, None, None
    dx, dw1, dw2, dw3 = grouped_swiglu_mxfp8_backward(dy, x, w1, w2, w3, counts, g, u, h, *quantized)
    return dx, dw1, dw2, dw3, None, None


grouped_swiglu_mxfp8.register_autograd(_gsmx_bwd, setup_context=_gsmx_setup)


# ---------------------------------------------------------------------------
# the routed half of MoE.forward with fp8 experts and the score applied before
# them, the permute folded into the token quantizers
# ---------------------------------------------------------------------------
def _aligned(src: Tensor) -> Tensor:
    return src.clone() if src.data_ptr() % 16 else src  # the gathering kernels read rows in 16-byte pieces


def _quant_rows_groupamax_gather(src: Tensor, token_idx: Tensor, row_scale: Tensor | None, counts: Tensor,
                                 e: int) -> tuple[Tensor, Tensor, Tensor]:
    """_quant_rows_groupamax of the routed rows src[token_idx] (* row_scale, rounded
    to bf16), read from src [N, C] in place."""
    src = _aligned(src)
    r, c = token_idx.shape[0], src.shape[1]
    q = torch.empty(r, c, dtype=FP8, device=src.device)
    sc = torch.empty(r, dtype=torch.float32, device=src.device)
    amax = torch.zeros(e, c, dtype=torch.float32, device=src.device)
    call("moe_fp8_quant_rows_groupamax_gather", ptr(src), src.shape[0], ptr(token_idx), ptr(row_scale), ptr(counts),
         r, e, c, ptr(q), ptr(sc), ptr(amax), stream_of(src))
    return q, sc, amax


def _quant_tokens_t_gather(src: Tensor, token_idx: Tensor, row_scale: Tensor | None, counts: Tensor, e: int,
                           rpad: int, amax: Tensor) -> tuple[Tensor, Tensor]:
    """_quant_tokens_t (from the groups' known amax) of the routed rows
    src[token_idx] (* row_scale, rounded to bf16), read from src in place."""
    src = _aligned(src)
    r, c = token_idx.shape[0], src.shape[1]
    q = torch.empty(c, rpad, dtype=FP8, device=src.device)
    sc = torch.empty(e, c, dtype=torch.float32, device=src.device)
    call("moe_fp8_quant_tokens_t_amax_gather", ptr(src), src.shape[0], ptr(token_idx), ptr(row_scale), ptr(amax),
         ptr(counts), r, e, c, rpad, ptr(q), ptr(sc), stream_of(src))
    return q, sc


@torch.library.custom_op("moe_mi355x::moe_core_fp8", mutates_args=())
def moe_core_fp8(
    x: Tensor, shared_out: Tensor | None, token_idx: Tensor, scores_sorted: Tensor, slot_pos: Tensor,
    tok_pos: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """out = combine(shared_out, experts(x[token_idx] * score)) with fp8 experts
    (moe.py:440-470 with score_before_experts; the ops of permute,
    grouped_swiglu_fp8 and combine): the routed rows are quantized straight from x
    (moe_fp8_quant_rows_groupamax_gather), so no routed copy of x is written, and
    in the backward the routed gradient and the routed x are quantized straight
    from the output's gradient and from x. Returns (out, g, u, h, then the column
    amax of w1, w3, w2, of the routed x and of h per token group)."""
    require_gpu(x, shared_out, token_idx, scores_sorted, slot_pos, tok_pos, w1, w2, w3, num_tokens_per_expert)
    _check_bf16("moe_core_fp8", x=x, w1=w1, w2=w2, w3=w3)
    x, w1, w2, w3 = x.contiguous(), w1.contiguous(), w2.contiguous(), w3.contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    tidx = token_idx.to(torch.int64).contiguous()
    sc = scores_sorted.float().contiguous()
    qx, sx, amx = _quant_rows_groupamax_gather(x, tidx, sc, counts, w1.shape[0])
    y, g, u, h, am1, am3, am2, amh = _fp8_experts_forward(qx, sx, w1, w2, w3, counts)
    out = combine(shared_out, y, slot_pos, tok_pos, None)
    return out, g, u, h, am1, am3, am2, amx, amh


@moe_core_fp8.register_fake
def _(x, shared_out, token_idx, scores_sorted, slot_pos, tok_pos, w1, w2, w3, num_tokens_per_expert):
    n, d = x.shape
    r = token_idx.shape[0]
    e, h_dim, _ = w1.shape
    f32 = lambda *shape: x.new_empty(*shape, dtype=torch.float32)  # noqa: E731
    return (x.new_empty(n, d), x.new_empty(r, h_dim), x.new_empty(r, h_dim), x.new_empty(r, h_dim),
            f32(*_amax_shape(e, d)), f32(*_amax_shape(e, d)), f32(*_amax_shape(e, h_dim)), f32(e, d),
            f32(*_amax_shape(e, h_dim)))


@torch.library.custom_op("moe_mi355x::moe_core_fp8_backward", mutates_args=())
def moe_core_fp8_backward(
    grad_out: Tensor, x: Tensor, token_idx: Tensor, scores_sorted: Tensor, tok_pos: Tensor, w1: Tensor,
    w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor, g: Tensor, u: Tensor, h: Tensor, amax_w1: Tensor,
    amax_w3: Tensor, amax_w2: Tensor, amax_x: Tensor, amax_h: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(grad_x, grad_scores_sorted, dw1, dw2, dw3) of moe_core_fp8's out; the
    shared output's gradient is grad_out itself (the combine adds it once)."""
    require_gpu(grad_out, x, token_idx, scores_sorted, tok_pos, w1, w2, w3, num_tokens_per_expert, g, u, h)
    go = grad_out.to(torch.bfloat16).contiguous()
    x = x.contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    tidx = token_idx.to(torch.int64).contiguous()
    sc = scores_sorted.float().contiguous()
    e = w1.shape[0]
    qdy, sdy, amdy = _quant_rows_groupamax_gather(go, tidx, None, counts, e)
    dx_routed, dw1, dw2, dw3 = _fp8_experts_backward(
        qdy, sdy, w1, w2, w3, counts, g, u, h, amax_w1, amax_w3, amax_w2, amax_h,
        lambda rpad: _quant_tokens_t_gather(x, tidx, sc, counts, e, rpad, amax_x),
        lambda rpad: _quant_tokens_t_gather(go, tidx, None, counts, e, rpad, amdy))
    grad_x, grad_s = permute_backward(dx_routed, x, tok_pos, scores_sorted, PERMUTE_BWD_ROUND_EACH)
    return grad_x, grad_s, dw1, dw2, dw3


@moe_core_fp8_backward.register_fake
def _(grad_out, x, token_idx, scores_sorted, tok_pos, w1, w2, w3, num_tokens_per_expert, *saved):
    r = token_idx.shape[0]
    return (x.new_empty(x.shape), x.new_empty(r, dtype=torch.float32), torch.empty_like(w1), torch.empty_like(w2),
            torch.empty_like(w3))


def _core_fp8_setup(ctx, inputs, output):
    x, shared_out, token_idx, scores_sorted, _slot_pos, tok_pos, w1, w2, w3, counts = inputs
    _out, g, u, h, *amax = output
    ctx.save_for_backward(x, token_idx, scores_sorted, tok_pos, w1, w2, w3, counts, g, u, h, *amax)
    ctx.has_shared = shared_out is not None
    ctx.shared_dtype = shared_out.dtype if shared_out is not None else None
    ctx.mark_non_differentiable(g, u, h, *amax)
    ctx.set_materialize_grads(False)


def _core_fp8_bwd(ctx, grad_out, *_unused):
    if grad_out is None:
        return (None,) * 10
    x, token_idx, scores_sorted, tok_pos, w1, w2, w3, counts, g, u, h, *amax = ctx.saved_tensors
    grad_x, grad_s, dw1, dw2, dw3 = moe_core_fp8_backward(grad_out, x, token_idx, scores_sorted, tok_pos, w1, w2,
                                                          w3, counts, g, u, h, *amax)
    grad_shared = grad_out.to(ctx.shared_dtype) if ctx.has_shared else None
    return grad_x, grad_shared, None, grad_s, None, None, dw1, dw2, dw3, None


moe_core_fp8.register_autograd(_core_fp8_bwd, setup_context=_core_fp8_setup)


# ---------------------------------------------------------------------------
# the routed half of MoE.forward with MXFP8 experts and the score applied before
# them, the permute folded into the token quantizer
# ---------------------------------------------------------------------------
def _mx_dual_tokens_gather(src: Tensor, token_idx: Tensor, row_scale: Tensor | None, counts: Tensor, e: int,
                           rpad: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """_mx_dual_tokens of the routed rows src[token_idx] (* row_scale, rounded to
    bf16), read from src [N, C] in place."""
    src = _aligned(src)
    r = token_idx.shape[0]
    c = src.shape[1]
    qr = torch.empty(r, c, dtype=FP8, device=src.device)
    sr = torch.empty(r, c // MX_BLOCK, dtype=torch.uint8, device=src.device)
    qt = torch.empty(c, rpad, dtype=FP8, device=src.device)
    st = torch.empty(rpad // MX_BLOCK, c, dtype=torch.uint8, device=src.device)
    call("moe_mxfp8_quant_dual_tokens_gather", ptr(src), src.shape[0], ptr(token_idx), ptr(row_scale), ptr(counts),
         r, e, c, rpad, ptr(qr), ptr(sr), ptr(qt), ptr(st), stream_of(src))
    return qr, sr, qt, st


@torch.library.custom_op("moe_mi355x::moe_core_mxfp8", mutates_args=())
def moe_core_mxfp8(
    x: Tensor, shared_out: Tensor | None, token_idx: Tensor, scores_sorted: Tensor, slot_pos: Tensor,
    tok_pos: Tensor, w1: Tensor, w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """out = combine(shared_out, experts(x[token_idx] * score)) with MXFP8 experts
    (moe.py:440-470 with score_before_experts; the ops of permute,
    grouped_swiglu_mxfp8 and combine): the routed rows are quantized straight from
    x (moe_mxfp8_quant_dual_tokens_gather), so no routed copy of x is written, and
    in the backward the routed gradient is quantized straight from the output's
    gradient. Returns (out, g, u, h, then the forward's quantized layouts the
    backward reuses)."""
    require_gpu(x, shared_out, token_idx, scores_sorted, slot_pos, tok_pos, w1, w2, w3, num_tokens_per_expert)
    _check_bf16("moe_core_mxfp8", x=x, w1=w1, w2=w2, w3=w3)
    x, w1, w2, w3 = x.contiguous(), w1.contiguous(), w2.contiguous(), w3.contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    tidx = token_idx.to(torch.int64).contiguous()
    sc = scores_sorted.float().contiguous()
    r = tidx.shape[0]
    d = x.shape[1]
    e, h_dim, _ = w1.shape
    s = stream_of(x)
    rpad = _mx_padded_rows(r, e)
    qx, sx, qxt, sxt = _mx_dual_tokens_gather(x, tidx, sc, counts, e, rpad)
    qw1, sw1, qw3, sw3, qw2, sw2, qw2t, sw2t, qw13t, sw13t = _mx_weights(w1, w2, w3, True)
    g = x.new_empty(r, h_dim)
    u = x.new_empty(r, h_dim)
    h = x.new_empty(r, h_dim)
    call("moe_mxfp8_gemm_gate_up", ptr(qx), ptr(sx), ptr(qw1), ptr(sw1), ptr(qw3), ptr(sw3), ptr(counts), r, e, d,
         h_dim, ptr(g), ptr(u), ptr(h), s)
    qh, sh, qht, sht = _mx_dual_tokens(h, counts, e, rpad)
    y = x.new_empty(r, d)
    call("moe_mxfp8_gemm_down", ptr(qh), ptr(sh), ptr(qw2), ptr(sw2), ptr(counts), r, e, d, h_dim, ptr(y), s)
    out = combine(shared_out, y, slot_pos, tok_pos, None)
    return out, g, u, h, qxt, sxt, qht, sht, qw2t, sw2t, qw13t, sw13t


@moe_core_mxfp8.register_fake
def _(x, shared_out, token_idx, scores_sorted, slot_pos, tok_pos, w1, w2, w3, num_tokens_per_expert):
    n, d = x.shape
    r = token_idx.shape[0]
    e, h_dim, _ = w1.shape
    u8 = lambda *shape: x.new_empty(*shape, dtype=torch.uint8)  # noqa: E731
    rpad = (r + e * 127 + 127) // 128 * 128  # _mx_padded_rows
    return (x.new_empty(n, d), x.new_empty(r, h_dim), x.new_empty(r, h_dim), x.new_empty(r, h_dim),
            u8(d, rpad), u8(rpad // 32, d), u8(h_dim, rpad), u8(rpad // 32, h_dim),
            u8(e, h_dim, d), u8(e, h_dim, d // 32), u8(e, d, 2 * h_dim), u8(e, d, 2 * h_dim // 32))


@torch.library.custom_op("moe_mi355x::moe_core_mxfp8_backward", mutates_args=())
def moe_core_mxfp8_backward(
    grad_out: Tensor, x: Tensor, token_idx: Tensor, scores_sorted: Tensor, tok_pos: Tensor, w1: Tensor,
    w2: Tensor, w3: Tensor, num_tokens_per_expert: Tensor, g: Tensor, u: Tensor, h: Tensor, qxt: Tensor,
    sxt: Tensor, qht: Tensor, sht: Tensor, qw2t: Tensor, sw2t: Tensor, qw13t: Tensor, sw13t: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(grad_x, grad_scores_sorted, dw1, dw2, dw3) of moe_core_mxfp8's out; the
    shared output's gradient is grad_out itself (the combine adds it once)."""
    require_gpu(grad_out, x, token_idx, scores_sorted, tok_pos, w1, w2, w3, num_tokens_per_expert, g, u, h)
    go = grad_out.to(torch.bfloat16).contiguous()
    counts = num_tokens_per_expert.to(torch.int64).contiguous()
    tidx = token_idx.to(torch.int64).contiguous()
    r = tidx.shape[0]
    d = x.shape[1]
    e = w1.shape[0]
    rpad = _mx_padded_rows(r, e)
    qdy = _mx_dual_tokens_gather(go, tidx, None, counts, e, rpad)
    dx_routed, dw1, dw2, dw3 = _mx_experts_backward(qdy, r, d, w1, w2, w3, counts, g, u, h, qxt, sxt, qht, sht,
                                                    qw2t, sw2t, qw13t, sw13t, rpad)
    grad_x, grad_s = permute_backward(dx_routed, x, tok_pos, scores_sorted, PERMUTE_BWD_ROUND_EACH)
    return grad_x, grad_s, dw1, dw2, dw3


@moe_core_mxfp8_backward.register_fake
def _(grad_out, x, token_idx, scores_sorted, tok_pos, w1, w2, w3, num_tokens_per_expert, *saved):
    r = token_idx.shape[0]
    return (x.new_empty(x.shape), x.new_empty(r, dtype=torch.float32), torch.empty_like(w1), torch.empty_like(w2),
            torch.empty_like(w3))


def _core_mx_setup(ctx, inputs, output):
    x, shared_out, token_idx, scores_sorted, _slot_pos, tok_pos, w1, w2, w3, counts = inputs
    _out, g, u, h, *quantized = output
    ctx.save_for_backward(x, token_idx, scores_sorted, tok_pos, w1, w2, w3, counts, g, u, h, *quantized)
    ctx.has_shared = shared_out is not None
    ctx.shared_dtype = shared_out.dtype if shared_out is not None else None
    ctx.mark_non_differentiable(g, u, h, *quantized)
    ctx.set_materialize_grads(False)


def _core_mx_bwd(ctx, grad_out, *_unused):
    if grad_out is None:
        return (None,) * 10
    x, token_idx, scores_sorted, tok_pos, w1, w2, w3, counts, g, u, h, *quantized = ctx.saved_tensors
    grad_x, grad_s, dw1, dw2, dw3 = moe_core_mxfp8_backward(grad_out, x, token_idx, scores_sorted, tok_pos, w1, w2,
                                                            w3, counts, g, u, h, *quantized)
    grad_shared = grad_out.to(ctx.shared_dtype) if ctx.has_shared else None
    return grad_x, grad_shared, None, grad_s, None, None, dw1, dw2, dw3, None


moe_core_mxfp8.register_autograd(_core_mx_bwd, setup_context=_core_mx_setup)


# ---------------------------------------------------------------------------
# row gather / scatter by an index (expert-parallel permute and unpermute)
# ---------------------------------------------------------------------------
@torch.library.custom_op("moe_mi355x::gather_rows", mutates_args=())
def gather_rows(src: Tensor, idx: Tensor) -> Tensor:
    """dst = src[idx, :] (expert_parallel.py:70-74)."""
    require_gpu(src, idx)
    s = src.contiguous()
    ix = idx.to(torch.int64).contiguous()
    n, d = ix.shape[0], s.shape[1]
    out = s.new_empty(n, d)
    call("moe_gather_rows", ptr(s), s.shape[0], ptr(ix), n, d, _dtype_code(s), ptr(out), stream_of(s))
    return out


@gather_rows.register_fake
def _(src, idx):
    return src.new_empty(idx.shape[0], src.shape[1])


@torch.library.custom_op("moe_mi355x::scatter_rows", mutates_args=())
def scatter_rows(src: Tensor, idx: Tensor, n_rows: int) -> Tensor:
    """dst = empty(n_rows, d); dst[idx, :] = src (expert_parallel.py:77-80). Rows of
    dst that idx does not name are left uninitialised, as in the reference."""
    require_gpu(src, idx)
    s = src.contiguous()
    ix = idx.to(torch.int64).contiguous()
    out = s.new_empty(n_rows, s.shape[1])
    call("moe_scatter_rows", ptr(s), ptr(ix), ix.shape[0], s.shape[1], _dtype_code(s), ptr(out), n_rows,
         stream_of(s))
    return out


@scatter_rows.register_fake
def _(src, idx, n_rows):
    return src.new_empty(n_rows, src.shape[1])


def _rows_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[1])
    ctx.n_src = inputs[0].shape[0]


def _gather_rows_bwd(ctx, g):
    # a permutation: every source row receives exactly one gradient row
    (idx,) = ctx.saved_tensors
    return scatter_rows(g, idx, ctx.n_src), None


def _scatter_rows_bwd(ctx, g):
    (idx,) = ctx.saved_tensors
    return gather_rows(g, idx), None, None


gather_rows.register_autograd(_gather_rows_bwd, setup_context=_rows_setup)
scatter_rows.register_autograd(_scatter_rows_bwd, setup_context=_rows_setup)
