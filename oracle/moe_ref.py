"""ORACLE — CPU restatement of torchtitan's MoE layer hot path. TEST INFRASTRUCTURE.

This module is the checker for the MI355X kernels. Only tests/, the smoke()
of __graft_entry__.py and bench.py's cpu_baseline leg may import it; the
product (torchtitan_amd) never does.

It restates the reference's algorithm (QIU023/torchtitan):
  torchtitan/models/common/moe.py:24-489       (router, reorderer, experts, MoE.forward)
  torchtitan/ops/scatter_add.py:10-48          (deterministic scatter_add + backward)
  torchtitan/models/common/feed_forward.py:34-54
  torchtitan/distributed/expert_parallel.py:26-67 (_generate_permute_indices)
  torchtitan/models/gpt_oss/moe.py:43-122      (gpt-oss experts)
with the GPU lowering of the ops the reference calls made explicit, because on
the GPU those are what define the reference's results:
  * torch.topk(sorted=False): radix order, lowest index first among ties, output
    slots = keys above the k-th key by ascending index, then k-th-key ties;
  * torch.sum over a short row: pairwise tree over adjacent lanes;
  * torch.histc(int64): bincount (the reference's CPU histc rejects int64);
  * deterministic scatter_add: starting from the destination row, add a token's
    rows in ascending position, rounding to the row dtype after every add
    (ATen's sorted index_put with accumulate);
  * x[token_idx] backward: accumulate in ascending position, rounding each add.
Those lowering claims are pinned by GPU tests that run the same torch ops on
the device (tests/test_gpu_oracle_pins.py); the arithmetic is pinned by closed
forms, brute force and finite differences (tests/test_oracle.py).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

# ---------------------------------------------------------------------------
# selection rules (numpy)
# ---------------------------------------------------------------------------


def radix_key(x: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 key of fp32 values: -0 < +0, NaN largest."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    mask = np.where(b & np.uint32(0x80000000), np.uint32(0xFFFFFFFF), np.uint32(0x80000000))
    k = b ^ mask
    return np.where(np.isnan(x), np.uint32(0xFFFFFFFF), k).astype(np.uint32)


def topk_gpu_order(values: np.ndarray, k: int) -> np.ndarray:
    """Indices of torch.topk(values, k, dim=-1, sorted=False) on the GPU
    (moe.py:199-201, :247-249): the k largest radix keys, lowest index first
    among equal keys; emitted as the entries whose key exceeds the k-th key in
    ascending index, then the k-th-key ties in ascending index."""
    v = np.asarray(values, dtype=np.float32)
    n, e = v.shape
    key = radix_key(v).astype(np.int64)
    # stable sort by key descending == ascending index among ties
    order = np.argsort(-key, axis=1, kind="stable")[:, :k]
    sel_key = np.take_along_axis(key, order, axis=1)
    kth = sel_key[:, k - 1 : k]
    cls = (sel_key <= kth).astype(np.int64)  # 0: above the k-th key, 1: tie with it
    comb = cls * (e + 1) + order
    out_rank = np.argsort(comb, axis=1, kind="stable")
    return np.take_along_axis(order, out_rank, axis=1).astype(np.int64)


def gpu_row_sum(v: torch.Tensor) -> torch.Tensor:
    """Sum over the last dim (size n <= 64) in torch's GPU reduction order for a
    short contiguous row: bw = largest power of two <= n; lane x forms
    v[x] + v[x+bw]; then lanes combine pairwise with offsets 1, 2, 4, ...
    Differentiable (plain torch indexing and adds)."""
    n = v.shape[-1]
    bw = 1
    while bw * 2 <= n:
        bw *= 2
    parts = []
    for x in range(bw):
        p = v[..., x]
        if x + bw < n:
            p = p + v[..., x + bw]
        parts.append(p)
    off = 1
    while off < bw:
        parts = [parts[i] + parts[i + off] if i % (2 * off) == 0 else parts[i] for i in range(bw)]
        off *= 2
    return parts[0]


def node_limited_choice(choice: np.ndarray, n_groups: int, n_limited: int) -> np.ndarray:
    """_get_node_limited_routing_scores (moe.py:169-209): group score = sum of the
    two largest scores in the group; keep the n_limited best groups
    (topk sorted=False rule); set the other groups' experts to -inf."""
    n, e = choice.shape
    epg = e // n_groups
    g = np.asarray(choice, dtype=np.float32).reshape(n, n_groups, epg)
    key = radix_key(g).astype(np.int64)
    top2 = np.argsort(-key, axis=2, kind="stable")[:, :, :2]
    vals = np.take_along_axis(g, top2, axis=2)
    group_scores = (vals[:, :, 0] + vals[:, :, 1]).astype(np.float32)
    keep = topk_gpu_order(group_scores, n_limited)
    mask = np.ones((n, n_groups), dtype=bool)
    np.put_along_axis(mask, keep, False, axis=1)
    out = np.where(mask[:, :, None], np.float32(-np.inf), g).astype(np.float32)
    return out.reshape(n, e)


# ---------------------------------------------------------------------------
# router (moe.py:211-276)
# ---------------------------------------------------------------------------


@dataclass
class RouterCfg:
    num_experts: int
    top_k: int
    score_func: str = "sigmoid"
    num_expert_groups: int | None = None
    num_limited_groups: int | None = None
    route_norm: bool = False
    route_scale: float = 1.0
    force_load_balance: bool = False


def score_fn(logits: torch.Tensor, score_func: str) -> torch.Tensor:
    """moe.py:236-241 (fp32)."""
    if score_func == "sigmoid":
        return torch.sigmoid(logits)
    if score_func == "softmax":
        return F.softmax(logits, dim=1)
    raise NotImplementedError(f"Unknown score function {score_func}")


def select_experts(scores: np.ndarray, expert_bias: np.ndarray | None, cfg: RouterCfg) -> np.ndarray:
    """Expert choice from fp32 scores (moe.py:243-261). Returns [N,K] int64."""
    n = scores.shape[0]
    if cfg.force_load_balance:
        return (np.arange(n * cfg.top_k, dtype=np.int64).reshape(n, cfg.top_k)) % cfg.num_experts
    choice = scores if expert_bias is None else (scores + expert_bias[None, :]).astype(np.float32)
    if cfg.num_expert_groups is not None:
        choice = node_limited_choice(choice, cfg.num_expert_groups, cfg.num_limited_groups)
    return topk_gpu_order(choice, cfg.top_k)


def router_forward(logits: torch.Tensor, expert_bias: torch.Tensor | None, cfg: RouterCfg,
                   scores: torch.Tensor | None = None):
    """Returns (top_scores [N,K] f32, idx [N,K] i64, counts [E] i64, scores [N,E] f32).
    `scores` may be supplied to route from given score-function outputs (to
    compare selection bit-exactly with a device that computed them)."""
    if scores is None:
        scores = score_fn(logits.float(), cfg.score_func)
    bias_np = expert_bias.detach().float().cpu().numpy() if expert_bias is not None else None
    idx_np = select_experts(scores.detach().cpu().numpy(), bias_np, cfg)
    idx = torch.from_numpy(idx_np).to(scores.device)
    top_scores = scores.gather(1, idx)
    if cfg.route_norm:
        den = gpu_row_sum(top_scores).unsqueeze(-1) + 1e-20
        top_scores = top_scores / den
    top_scores = top_scores * cfg.route_scale
    counts = torch.bincount(idx.view(-1), minlength=cfg.num_experts)
    return top_scores, idx, counts, scores


# ---------------------------------------------------------------------------
# reorderer (moe.py:291-332) and EP permute indices (expert_parallel.py:26-67)
# ---------------------------------------------------------------------------


def reorder(top_scores: torch.Tensor, idx: torch.Tensor, num_experts: int):
    """(scores_sorted [R], token_idx [R] i64, counts [E] i64, perm [R] i64)."""
    k = idx.shape[1]
    flat = idx.reshape(-1)
    counts = torch.bincount(flat, minlength=num_experts)
    perm = torch.from_numpy(np.argsort(flat.cpu().numpy(), kind="stable")).to(flat.device)
    scores_sorted = top_scores.reshape(-1)[perm]
    return scores_sorted, perm // k, counts, perm


def generate_permute_indices(tokens_per_expert_group, experts_per_rank: int, num_ranks: int):
    """Rank-major -> expert-major gather indices (expert_parallel.py:26-67)."""
    t = np.asarray(tokens_per_expert_group, dtype=np.int64)
    mat = t.reshape(num_ranks, experts_per_rank)
    in_start = (np.cumsum(t) - t).reshape(num_ranks, experts_per_rank)
    seg_len = mat.T.reshape(-1)
    seg_in = in_start.T.reshape(-1)
    seg_out = np.cumsum(seg_len) - seg_len
    out = np.empty(int(t.sum()), dtype=np.int64)
    for s in range(seg_len.shape[0]):
        n = int(seg_len[s])
        out[seg_out[s] : seg_out[s] + n] = seg_in[s] + np.arange(n)
    return out, mat.sum(axis=0)


def generate_permute_pad_indices(tokens_per_expert_group, experts_per_rank: int, num_ranks: int, pad: int):
    """The permute_and_pad layout TorchAOExpertParallel relies on
    (expert_parallel.py:537-562; torchao's permute_and_pad itself is absent, so this
    is fixed by its call site): the rows of generate_permute_indices, each expert's
    group followed by zero rows up to a multiple of `pad`; padding rows index the
    extra zero row appended after the input (index sum(counts), dropped again by
    _unpermute's [:-1]). Returns (indices, padded counts, inclusive group ends)."""
    idx, per_expert = generate_permute_indices(tokens_per_expert_group, experts_per_rank, num_ranks)
    n_in = int(np.asarray(tokens_per_expert_group).sum())
    out, padded, ends, pos = [], [], [], 0
    for e in range(experts_per_rank):
        g = int(per_expert[e])
        gp = (g + pad - 1) // pad * pad
        out.extend(idx[pos : pos + g].tolist())
        out.extend([n_in] * (gp - g))
        pos += g
        padded.append(gp)
        ends.append((ends[-1] if ends else 0) + gp)
    return np.asarray(out, dtype=np.int64), np.asarray(padded, dtype=np.int64), np.asarray(ends, dtype=np.int64)


def expert_bias_update(tokens_per_expert, expert_bias, coeffs, halve) -> None:
    """_update_expert_bias, torchtitan/components/optimizer.py:386-431, per layer
    with the same torch ops: t = tokens_per_expert (// 2 for recomputing blocks),
    delta = coeff * sign(mean(t) - t), delta -= mean(delta), expert_bias += delta,
    tokens_per_expert = 0. Updates the tensors in place."""
    with torch.no_grad():
        for t, b, c, hv in zip(tokens_per_expert, expert_bias, coeffs, halve):
            tt = (t // 2 if hv else t).float()
            delta = c * torch.sign(tt.mean() - tt)
            delta = delta - delta.mean()
            b.add_(delta)
            t.zero_()


# ---------------------------------------------------------------------------
# row movement with the GPU accumulation semantics
# ---------------------------------------------------------------------------


class _IndexRows(torch.autograd.Function):
    """routed = x[token_idx] (moe.py:445); backward accumulates each token's rows
    in ascending position, rounding to x's dtype after every add."""

    @staticmethod
    def forward(ctx, x, token_idx):
        ctx.save_for_backward(token_idx)
        ctx.n = x.shape[0]
        return x[token_idx]

    @staticmethod
    def backward(ctx, g):
        (token_idx,) = ctx.saved_tensors
        return index_backward(g, token_idx, ctx.n), None


def index_backward(g: torch.Tensor, token_idx: torch.Tensor, n: int) -> torch.Tensor:
    dtype = g.dtype
    order = torch.from_numpy(np.argsort(token_idx.cpu().numpy(), kind="stable"))
    t_sorted = token_idx[order]
    counts = torch.bincount(token_idx, minlength=n)
    maxk = int(counts.max().item()) if counts.numel() else 0
    acc = torch.zeros(n, g.shape[1], dtype=torch.float32)
    start = torch.cumsum(counts, 0) - counts
    rank = torch.arange(order.numel()) - start[t_sorted]
    for j in range(maxk):
        sel = rank == j
        rows = order[sel]
        toks = t_sorted[sel]
        acc[toks] = (acc[toks] + g[rows].float()).to(dtype).float()
    return acc.to(dtype)


class _Combine(torch.autograd.Function):
    """deterministic_scatter_add(out, token_idx expanded, src) (scatter_add.py:10-48):
    starting from out[t], each of token t's rows is added in ascending position
    with a rounding to out's dtype after every add. Backward: grad passes to out;
    grad_src = gather."""

    @staticmethod
    def forward(ctx, out, token_idx, src):
        ctx.save_for_backward(token_idx)
        dtype = out.dtype
        acc = out.float().clone()
        order = torch.from_numpy(np.argsort(token_idx.cpu().numpy(), kind="stable"))
        t_sorted = token_idx[order]
        counts = torch.bincount(token_idx, minlength=out.shape[0])
        start = torch.cumsum(counts, 0) - counts
        rank = torch.arange(order.numel()) - start[t_sorted]
        maxk = int(counts.max().item()) if counts.numel() else 0
        for j in range(maxk):
            sel = rank == j
            toks = t_sorted[sel]
            acc[toks] = (acc[toks] + src[order[sel]].float()).to(dtype).float()
        return acc.to(dtype)

    @staticmethod
    def backward(ctx, g):
        (token_idx,) = ctx.saved_tensors
        return g, None, g[token_idx]


# ---------------------------------------------------------------------------
# experts (moe.py:24-70) and the shared expert (feed_forward.py:53-54)
# ---------------------------------------------------------------------------


def experts_grouped_mm(w1, w2, w3, x, counts):
    """_run_experts_grouped_mm: bf16 per-segment GEMMs, fp32 accumulate, bf16
    outputs, each bf16 elementwise op rounded (moe.py:53-70). Uses per-segment
    matmuls, which is what torch._grouped_mm computes per group."""
    xb, w1b, w2b, w3b = x.bfloat16(), w1.bfloat16(), w2.bfloat16(), w3.bfloat16()
    outs = []
    start = 0
    for e, c in enumerate(counts.tolist()):
        xe = xb[start : start + c]
        g = (xe.float() @ w1b[e].float().t()).bfloat16()
        u = (xe.float() @ w3b[e].float().t()).bfloat16()
        h = F.silu(g) * u
        outs.append((h.float() @ w2b[e].float().t()).bfloat16())
        start += c
    tail = xb.new_zeros(xb.shape[0] - start, w2.shape[1])
    return torch.cat(outs + [tail], 0).type_as(x)


def experts_for_loop(w1, w2, w3, x, counts):
    """_run_experts_for_loop (moe.py:24-50): matmuls in the input dtype."""
    outs = []
    start = 0
    for e, c in enumerate(counts.tolist()):
        xe = x[start : start + c]
        h = F.silu(xe @ w1[e].t()) * (xe @ w3[e].t())
        outs.append(h @ w2[e].t())
        start += c
    return torch.cat(outs, 0)


# ---------------------------------------------------------------------------
# gpt-oss experts (torchtitan/models/gpt_oss/moe.py:43-122)
# ---------------------------------------------------------------------------

OSS_ALPHA = 1.702


def oss_swiglu(h1: torch.Tensor, limit: float, alpha: float = OSS_ALPHA) -> torch.Tensor:
    """swiglu (gpt_oss/moe.py:43-52) on an interleaved [.., 2H] tensor: glu =
    even columns clamped above at limit, linear = odd columns clamped to
    [-limit, limit]; glu * sigmoid(alpha glu) * (linear + 1), in h1's dtype."""
    x_glu, x_linear = h1[..., ::2], h1[..., 1::2]
    x_glu = x_glu.clamp(min=None, max=limit)
    x_linear = x_linear.clamp(min=-limit, max=limit)
    out_glu = x_glu * torch.sigmoid(alpha * x_glu)
    return out_glu * (x_linear + 1)


def oss_experts_grouped_mm(mlp1_weight, mlp1_bias, mlp2_weight, mlp2_bias, limit, x, counts, aux=None):
    """The grouped-mm path (gpt_oss/moe.py:92-122) with the reference's torch
    calls: torch._grouped_mm over int32 offsets, biases broadcast per row with
    repeat_interleave (plus the zero row for rows past the groups) and added in
    bf16, then the clamped SwiGLU and the second grouped GEMM. With `aux`, the
    biased h1 and the output keep their gradients (aux["h1"], aux["y"]): the
    rows whose per-expert sums are the bias gradients."""
    offsets = torch.cumsum(counts, dim=0, dtype=torch.int32)
    tail = (x.shape[0] - offsets[-1]).unsqueeze(0).to(counts.dtype)
    counts_long = torch.cat([counts, tail]).long()
    h = torch._grouped_mm(x.bfloat16(), mlp1_weight.transpose(-2, -1).bfloat16(), offs=offsets)
    b1 = torch.cat([mlp1_bias, mlp1_bias.new_zeros(1, mlp1_bias.shape[-1])])
    b1 = b1.repeat_interleave(counts_long, dim=0, output_size=x.shape[0])
    h = h + b1.to(h.dtype)
    if aux is not None and h.requires_grad:
        h.retain_grad()
        aux["h1"] = h
    h = oss_swiglu(h, limit)
    h = torch._grouped_mm(h, mlp2_weight.transpose(-2, -1).bfloat16(), offs=offsets)
    b2 = torch.cat([mlp2_bias, mlp2_bias.new_zeros(1, mlp2_bias.shape[-1])])
    b2 = b2.repeat_interleave(counts_long, dim=0, output_size=x.shape[0])
    y = h + b2.to(h.dtype)
    if aux is not None and y.requires_grad:
        y.retain_grad()
        aux["y"] = y
    return y


def oss_experts_for_loop(mlp1_weight, mlp1_bias, mlp2_weight, mlp2_bias, limit, x, counts):
    """The for-loop path (gpt_oss/moe.py:55-89): matmuls in x's dtype."""
    outs, start = [], 0
    for e, c in enumerate(counts.tolist()):
        xe = x[start:start + c]
        h = xe @ mlp1_weight[e].transpose(-2, -1) + mlp1_bias[e]
        h = oss_swiglu(h, limit)
        outs.append(h @ mlp2_weight[e].transpose(-2, -1) + mlp2_bias[e])
        start += c
    return torch.cat(outs, 0)


def feed_forward(x, w1, w2, w3):
    return F.linear(F.silu(F.linear(x, w1)) * F.linear(x, w3), w2)


# ---------------------------------------------------------------------------
# the gate's backward on bf16 GEMMs (a re-expression of the fp32 autocast
# backward of moe.py:229-232; exact products, fp32 accumulation)
# ---------------------------------------------------------------------------


def gate_grad_split3(d: torch.Tensor) -> torch.Tensor:
    """[N, C] fp32 -> [N, 3C] bf16 (hi | mid | lo) with hi + mid + lo == d: each
    term takes the next 8 significand bits of what the previous ones left, so
    three cover fp32's 24 (torch casts, round to nearest even)."""
    hi = d.bfloat16()
    r = d - hi.float()
    mid = r.bfloat16()
    lo = (r - mid.float()).bfloat16()
    return torch.cat([hi, mid, lo], dim=1)


def gate_dw_reduce(partials: torch.Tensor, num_experts: int) -> torch.Tensor:
    """fp32 partials of terms^T x, [3E, D] or [2, 3E, D] (two token halves) ->
    dW [E, D] bf16: the halves added, then (hi + mid) + lo, rounded once."""
    p = partials.float()
    if p.dim() == 3:
        p = p[0] + p[1]
    e = num_experts
    return ((p[:e] + p[e:2 * e]) + p[2 * e:]).bfloat16()


# ---------------------------------------------------------------------------
# MoE.forward (moe.py:380-477)
# ---------------------------------------------------------------------------


@dataclass
class MoECfg:
    router: RouterCfg
    dim: int
    hidden_dim: int
    score_before_experts: bool = True
    use_grouped_mm: bool = True
    has_shared: bool = False
    # "swiglu"; "gptoss" (gpt_oss/moe.py GptOssGroupedExperts); "fp8" / "mxfp8": the
    # SwiGLU experts on the fp8 or MXFP8 emulations below (forward only)
    expert_kind: str = "swiglu"
    swiglu_limit: float = 7.0


def moe_forward(params: dict, x: torch.Tensor, cfg: MoECfg, aux: dict | None = None,
                logits: torch.Tensor | None = None):
    """params: 'gate' [E,D], 'w1','w2','w3' experts, optional 'sw1','sw2','sw3'
    shared expert, optional 'expert_bias' [E]. Records intermediates in `aux`.
    `logits` may carry the gate output computed elsewhere (the GPU's fp32 GEMM)
    so that both sides route from the same bits."""
    bs, slen, dim = x.shape
    x2 = x.reshape(-1, dim)
    gate_out = F.linear(x2.float(), params["gate"].float())  # fp32 gate (autocast on GPU)
    if logits is None:
        logits = gate_out
    else:
        # the given values (x - x == 0 exactly), with the gradient of the gate GEMM
        logits = logits.to(gate_out.dtype) + (gate_out - gate_out.detach())
    top_scores, idx, counts, scores = router_forward(logits, params.get("expert_bias"), cfg.router)
    scores_sorted, token_idx, counts2, perm = reorder(top_scores, idx, cfg.router.num_experts)
    routed_input = _IndexRows.apply(x2, token_idx)
    if cfg.score_before_experts:
        routed_input = (routed_input.float() * scores_sorted.reshape(-1, 1)).to(x2.dtype)
    run = experts_grouped_mm if cfg.use_grouped_mm else experts_for_loop
    routed_output = run(params["w1"], params["w2"], params["w3"], routed_input, counts2)
    if cfg.has_shared:
        out = feed_forward(x2, params["sw1"], params["sw2"], params["sw3"])
    else:
        out = torch.zeros_like(x2)
    if not cfg.score_before_experts:
        routed_output = (routed_output.float() * scores_sorted.reshape(-1, 1)).to(x2.dtype)
    out = _Combine.apply(out, token_idx, routed_output)
    if aux is not None:
        aux.update(logits=logits, scores=scores, top_scores=top_scores, idx=idx, counts=counts,
                   scores_sorted=scores_sorted, token_idx=token_idx, perm=perm,
                   routed_input=routed_input, routed_output=routed_output)
    return out.reshape(bs, slen, dim)


# ---------------------------------------------------------------------------
# the reference's router op sequence in plain torch ops (device-agnostic)
# ---------------------------------------------------------------------------


def router_forward_torch(logits: torch.Tensor, expert_bias: torch.Tensor | None, cfg: RouterCfg):
    """moe.py:236-274 op for op. Run on the GPU it is the reference router after
    the gate; the GPU tests use it to pin the selection / summation rules that
    router_forward restates. (histc on int64 is GPU-only, so counts use it only
    off the CPU.)"""
    # the score function runs in the gate's output dtype: fp32 on the GPU
    # (autocast), the input dtype on the CPU, as in the reference
    scores = score_fn(logits, cfg.score_func)
    choice = scores if expert_bias is None else scores + expert_bias
    if cfg.num_expert_groups is not None:
        g, gk = cfg.num_expert_groups, cfg.num_limited_groups
        grouped = choice.view(-1, g, cfg.num_experts // g)
        top2, _ = grouped.topk(2, dim=-1)
        group_scores = top2.sum(dim=-1)
        _, group_idx = torch.topk(group_scores, k=gk, dim=-1, sorted=False)
        group_mask = torch.ones_like(group_scores, dtype=torch.bool)
        group_mask.scatter_(1, group_idx, False)
        choice = grouped.masked_fill(group_mask.unsqueeze(-1), float("-inf")).view(-1, cfg.num_experts)
    _, idx = torch.topk(choice, k=cfg.top_k, dim=-1, sorted=False)
    top_scores = scores.gather(dim=1, index=idx)
    if cfg.force_load_balance:
        n = scores.shape[0]
        idx = torch.arange(n * cfg.top_k, device=scores.device, dtype=torch.int64).reshape(n, cfg.top_k)
        idx = idx % cfg.num_experts
        top_scores = scores.gather(dim=1, index=idx)
    if cfg.route_norm:
        top_scores = top_scores / (top_scores.sum(dim=-1, keepdim=True) + 1e-20)
    top_scores = top_scores * cfg.route_scale
    if logits.device.type == "cpu":
        counts = torch.bincount(idx.view(-1), minlength=cfg.num_experts)
    else:
        counts = torch.histc(idx.view(-1), bins=cfg.num_experts, min=0, max=cfg.num_experts)
    return top_scores, idx, counts, scores


# ---------------------------------------------------------------------------
# MoE.forward as the reference's own op sequence (device-agnostic)
# ---------------------------------------------------------------------------


def _histc_counts(flat_idx: torch.Tensor, num_experts: int) -> torch.Tensor:
    """moe.py:269-274 / :312-317. torch.histc rejects int64 on the CPU, so the
    CPU run uses bincount, which is the same histogram for ids in [0, E)."""
    if flat_idx.device.type == "cpu":
        return torch.bincount(flat_idx, minlength=num_experts)
    return torch.histc(flat_idx, bins=num_experts, min=0, max=num_experts)


def _deterministic_scatter_add(out: torch.Tensor, index: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """torchtitan/ops/scatter_add.py:10-20 (forward; autograd through ATen's
    scatter_add gives the same gather backward as :28-33)."""
    prev = torch.are_deterministic_algorithms_enabled()
    prev_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    torch.use_deterministic_algorithms(True, warn_only=False)
    try:
        return out.scatter_add(dim=0, index=index, src=src)
    finally:
        torch.use_deterministic_algorithms(prev, warn_only=prev_warn)


def moe_forward_reference_ops(params: dict, x: torch.Tensor, cfg: MoECfg, aux: dict | None = None,
                              logit_values: torch.Tensor | None = None) -> torch.Tensor:
    """MoE.forward (moe.py:380-477) with the router (moe.py:211-274), the
    reorderer (moe.py:291-332), _run_experts_grouped_mm (moe.py:53-70) and the
    shared FeedForward (feed_forward.py:53-54) written as the same torch calls
    the reference makes, so that it runs wherever torch does:
      * the gate runs under torch.autocast(dtype=float32) as at moe.py:231-232
        (honoured on the GPU, disabled with a warning on the CPU);
      * torch.histc on the GPU, bincount on the CPU (_histc_counts);
      * torch._grouped_mm in bf16, or the per-expert matmul loop when
        cfg.use_grouped_mm is False.
    This is the reference's CPU MoE path used as the CPU baseline, and, run on
    the GPU, the op-for-op reference the fused kernels are compared against.

    logit_values ([N, E] fp32, optional) replaces the values of the gate logits
    while their gradient still flows through the autocast gate: a caller whose
    logits differ from this GEMM's by fp32 summation order routes both sides on
    the same values (the difference is asserted to be that small)."""
    rc = cfg.router
    bs, slen, dim = x.shape
    x2 = x.view(-1, dim)
    gate_w = params["gate"]
    import warnings

    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        with torch.autocast(device_type=x.device.type, dtype=torch.float32):
            logits = F.linear(x2, gate_w, params.get("gate_bias"))
    if logit_values is not None:
        fix = logit_values.detach().float()
        d = fix - logits.detach()
        tol = 1e-5 * logits.detach().abs().max().clamp_min(1e-30)
        if not bool(d.abs().max() <= tol):
            raise AssertionError(f"logit_values differ from the fp32 gate GEMM by {d.abs().max().item():.3e}")
        logits = logits + d
        if not torch.equal(logits.detach(), fix):
            raise AssertionError("logit_values not reproduced exactly")
    top_scores, idx, _counts, _scores = router_forward_torch(logits, params.get("expert_bias"), rc)
    flat = idx.view(-1)
    counts = _histc_counts(flat, rc.num_experts)
    perm = torch.argsort(flat, stable=True)
    scores_sorted = top_scores.view(-1)[perm]
    token_idx = perm // rc.top_k
    routed_input = x2[token_idx]
    if cfg.score_before_experts:
        routed_input = (routed_input.to(torch.float32) * scores_sorted.reshape(-1, 1)).to(x2.dtype)
    if cfg.expert_kind == "gptoss":
        run = oss_experts_grouped_mm if cfg.use_grouped_mm else oss_experts_for_loop
        kw = {"aux": aux} if cfg.use_grouped_mm else {}
        routed_output = run(params["mlp1_weight"], params["mlp1_bias"], params["mlp2_weight"], params["mlp2_bias"],
                            cfg.swiglu_limit, routed_input, counts, **kw)
        if aux is not None:
            aux["counts"] = counts
    elif cfg.expert_kind in ("fp8", "mxfp8"):
        # the experts as the float8 / MXFP8 converters swap them in (torchao's grouped
        # GEMMs, restated by experts_fp8_forward / experts_mxfp8_forward); forward only
        run = experts_fp8_forward if cfg.expert_kind == "fp8" else experts_mxfp8_forward
        routed_output = run(params["w1"], params["w2"], params["w3"], routed_input.bfloat16(), counts)[0]
        routed_output = routed_output.type_as(routed_input)
    elif cfg.use_grouped_mm:
        w1, w2, w3 = params["w1"], params["w2"], params["w3"]
        offsets = torch.cumsum(counts, dim=0, dtype=torch.int32)
        h = F.silu(torch._grouped_mm(routed_input.bfloat16(), w1.bfloat16().transpose(-2, -1), offs=offsets))
        h = h * torch._grouped_mm(routed_input.bfloat16(), w3.bfloat16().transpose(-2, -1), offs=offsets)
        routed_output = torch._grouped_mm(h, w2.bfloat16().transpose(-2, -1), offs=offsets).type_as(routed_input)
    else:
        routed_output = experts_for_loop(params["w1"], params["w2"], params["w3"], routed_input, counts)
    if cfg.has_shared:
        out = feed_forward(x2, params["sw1"], params["sw2"], params["sw3"])
    else:
        out = torch.zeros_like(x2)
    if not cfg.score_before_experts:
        routed_output = (routed_output.to(torch.float32) * scores_sorted.reshape(-1, 1)).to(x2.dtype)
    out = _deterministic_scatter_add(out, token_idx.reshape(-1, 1).expand(-1, dim), routed_output)
    return out.reshape(bs, slen, dim)


# ---------------------------------------------------------------------------
# fp8 e4m3 grouped GEMMs (parity unpinned against torchao: the reference delegates
# to torchao's Float8TrainingOpConfig, torchtitan/components/quantization/float8.py:260-288,
# which is absent; this restates its rowwise recipe with power-of-two scales. The
# scale and cast are pinned by hand-worked scales and an independent e4m3 encoder,
# the expert GEMMs by e4m3-grid operands whose products must be exact, with
# planted scale-axis mistakes that those pins catch, in tests/test_oracle.py)
# ---------------------------------------------------------------------------

FP8_MAX = 448.0  # largest finite float8_e4m3fn
FP8_PAD = 16  # token-group alignment for fp8 grouped GEMMs (quantization/__init__.py:37-40)


def fp8_scale(amax: torch.Tensor) -> torch.Tensor:
    """Rowwise float8 scale of torchao's MoE training (torchao nightly, not vendored:
    prototype/moe_training `_Float8GroupedMM` calls float8_utils.tensor_to_scale
    with round_scales_to_power_of_2=True): m = fp32(448 / max(amax, 1e-12))
    formed in fp64, rounded down to a power of two 2^j. Returns the dequantization
    multiplier s = 2^-j (torchao passes the reciprocal of its scale to the GEMM).
    floor(log2 m) is taken from m's exponent; for bf16 inputs m is a power of two
    or at least 2^-9 below the next one, so a log2-based floor gives the same j."""
    m = (FP8_MAX / amax.double().clamp_min(1e-12)).float()
    _, e = torch.frexp(m)
    return torch.ldexp(torch.ones_like(m), (1 - e).float())


def quant_fp8_rows(x: torch.Tensor, dim: int = -1):
    """Dynamic fp8 quantization with one scale per slice along `dim`:
    s = fp8_scale(amax), q = e4m3fn(x / s) (x / s is exact, |x / s| <= 448;
    round to nearest even), which is torchao's to_fp8_saturated(x * 2^j).
    Returns (q float8_e4m3fn, s fp32 with `dim` kept as size 1)."""
    xf = x.float()
    amax = xf.abs().amax(dim=dim, keepdim=True)
    s = fp8_scale(amax)
    q = (xf / s).to(torch.float8_e4m3fn)
    return q, s


def _fp8_mm(qa, sa, qb, sb):
    """(qa @ qb^T) accumulated in fp64 then scaled as (acc * sa) * sb in fp32."""
    acc = (qa.double() @ qb.double().t()).float()
    return (acc * sa) * sb.reshape(1, -1)


def experts_fp8_forward(w1, w2, w3, x, counts):
    """fp8 forward of _run_experts_grouped_mm (moe.py:53-70): x and h quantized
    per token row, each weight per output row (per expert column), fp32
    accumulate, outputs g, u, h, y rounded to bf16 at the reference's points."""
    qx, sx = quant_fp8_rows(x)
    qw1, sw1 = quant_fp8_rows(w1)
    qw3, sw3 = quant_fp8_rows(w3)
    qw2, sw2 = quant_fp8_rows(w2)
    gs, us, hs = [], [], []
    start = 0
    for e, c in enumerate(counts.tolist()):
        sl = slice(start, start + c)
        g = _fp8_mm(qx[sl], sx[sl], qw1[e], sw1[e]).bfloat16()
        u = _fp8_mm(qx[sl], sx[sl], qw3[e], sw3[e]).bfloat16()
        gs.append(g); us.append(u); hs.append(F.silu(g) * u)
        start += c
    g, u, h = torch.cat(gs), torch.cat(us), torch.cat(hs)
    qh, sh = quant_fp8_rows(h)
    ys = []
    start = 0
    for e, c in enumerate(counts.tolist()):
        sl = slice(start, start + c)
        ys.append(_fp8_mm(qh[sl], sh[sl], qw2[e], sw2[e]).bfloat16())
        start += c
    return torch.cat(ys), g, u, h


def experts_fp8_backward(w1, w2, w3, x, counts, g, u, h, dy):
    """fp8 backward matching experts_fp8_forward: dh = dy . w2 with dy per row and
    w2 per (expert, h) column over D; SwiGLU backward in bf16; dx = bf16(dg . w1)
    + bf16(du . w3) with dg, du per row and w1, w3 per (expert, d) column over H;
    dw = per-group products over the expert's tokens with both operands scaled
    per (group, column) over those tokens."""
    E, H, D = w1.shape
    qdy, sdy = quant_fp8_rows(dy)
    dgs, dus = [], []
    start = 0
    for e, c in enumerate(counts.tolist()):
        sl = slice(start, start + c)
        qw2t, sw2t = quant_fp8_rows(w2[e].t())  # [H, D] rows
        dh = _fp8_mm(qdy[sl], sdy[sl], qw2t, sw2t).bfloat16()
        gg, uu = g[sl], u[sl]
        sl_g = F.silu(gg)
        dsl = (dh * uu)  # bf16 op: grad of silu output
        du = dh * sl_g
        dg = torch.ops.aten.silu_backward(dsl, gg)
        dgs.append(dg); dus.append(du)
        start += c
    dg, du = torch.cat(dgs), torch.cat(dus)
    qdg, sdg = quant_fp8_rows(dg)
    qdu, sdu = quant_fp8_rows(du)
    dxs, dw1s, dw2s, dw3s = [], [], [], []
    start = 0
    for e, c in enumerate(counts.tolist()):
        sl = slice(start, start + c)
        qw1t, sw1t = quant_fp8_rows(w1[e].t())  # [D, H]
        qw3t, sw3t = quant_fp8_rows(w3[e].t())
        dx = (_fp8_mm(qdg[sl], sdg[sl], qw1t, sw1t).bfloat16() + _fp8_mm(qdu[sl], sdu[sl], qw3t, sw3t).bfloat16())
        dxs.append(dx)
        if c == 0:
            dw1s.append(torch.zeros_like(w1[e])); dw3s.append(torch.zeros_like(w3[e])); dw2s.append(torch.zeros_like(w2[e]))
        else:
            qdgt, sdgt = quant_fp8_rows(dg[sl].t())  # [H, c]
            qdut, sdut = quant_fp8_rows(du[sl].t())
            qxt, sxt = quant_fp8_rows(x[sl].t())     # [D, c]
            qdyt, sdyt = quant_fp8_rows(dy[sl].t())  # [D, c]
            qht, sht = quant_fp8_rows(h[sl].t())     # [H, c]
            dw1s.append(_fp8_mm(qdgt, sdgt, qxt, sxt).bfloat16())
            dw3s.append(_fp8_mm(qdut, sdut, qxt, sxt).bfloat16())
            dw2s.append(_fp8_mm(qdyt, sdyt, qht, sht).bfloat16())
        start += c
    return torch.cat(dxs), torch.stack(dw1s), torch.stack(dw2s), torch.stack(dw3s)


# ---------------------------------------------------------------------------
# MXFP8 grouped GEMMs (parity unpinned: the reference delegates to torchao's
# MXFP8TrainingOpConfig, recipe "mxfp8_rceil", through MXFP8Converter,
# torchtitan/components/quantization/mx.py:25-128, and torchao is absent;
# this restates torchao's published to_mx with the RCEIL scale derivation)
# ---------------------------------------------------------------------------

MX_BLOCK = 32  # elements per e8m0 scale
MXFP8_PAD = 32  # token-group alignment (quantization/__init__.py:36-40)
E8M0_BIAS = 127


def quant_mxfp8(x: torch.Tensor, dim: int = -1):
    """MX quantization along `dim` in blocks of 32 (RCEIL):
    e = clamp(ceil(log2(amax / 448)), -127, 127) + 127 (255 where amax / 448
    is NaN), q = e4m3fn(clamp(x * m, -448, 448)) with m = 2^(127 - e), or
    m = 1 where e == 0. Returns (q float8_e4m3fn, e uint8 with `dim` / 32)."""
    xf = x.float().movedim(dim, -1)
    shp = xf.shape
    if shp[-1] % MX_BLOCK:
        raise ValueError(f"dimension {dim} ({shp[-1]}) is not a multiple of {MX_BLOCK}")
    blocks = xf.reshape(*shp[:-1], shp[-1] // MX_BLOCK, MX_BLOCK)
    amax = blocks.abs().amax(-1, keepdim=True)
    descale = amax / FP8_MAX
    e = torch.where(torch.isnan(descale), torch.full_like(descale, 255.0),
                    torch.clamp(torch.ceil(torch.log2(descale)), -E8M0_BIAS, E8M0_BIAS) + E8M0_BIAS)
    mult = torch.where(e == 0, torch.ones_like(e), torch.ldexp(torch.ones_like(e), (E8M0_BIAS - e)))
    q = torch.clamp(blocks * mult, -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.reshape(shp).movedim(-1, dim), e.squeeze(-1).to(torch.uint8).movedim(-1, dim)


def mx_dequant(q: torch.Tensor, e: torch.Tensor) -> torch.Tensor:
    """fp64 values q * 2^(e - 127) of an MX tensor quantized along its last dim."""
    f = torch.ldexp(torch.ones(e.shape, dtype=torch.float64, device=e.device), e.to(torch.float64) - E8M0_BIAS)
    return q.double() * f.repeat_interleave(MX_BLOCK, dim=-1)


def _mx_mm(qa, sa, qb, sb):
    """MX grouped-GEMM block: dequant(qa) @ dequant(qb)^T accumulated in fp64,
    returned as fp32 (both operands quantized along the contraction)."""
    return (mx_dequant(qa, sa) @ mx_dequant(qb, sb).t()).float()


def _pad_tokens(t: torch.Tensor, mult: int = MXFP8_PAD) -> torch.Tensor:
    """Zero-pads the last dimension (a token group) to a multiple of `mult`."""
    n = t.shape[-1]
    pad = (n + mult - 1) // mult * mult - n
    return torch.nn.functional.pad(t, (0, pad)) if pad else t


def experts_mxfp8_forward(w1, w2, w3, x, counts):
    """MXFP8 forward of _run_experts_grouped_mm (moe.py:53-70): x, h and every
    weight quantized in 32-blocks along the contraction, fp32 accumulation,
    g, u, h, y rounded to bf16 at the reference's points."""
    qx, sx = quant_mxfp8(x)
    qw1, sw1 = quant_mxfp8(w1)
    qw3, sw3 = quant_mxfp8(w3)
    qw2, sw2 = quant_mxfp8(w2)
    gs, us, hs = [], [], []
    start = 0
    for e, c in enumerate(counts.tolist()):
        sl = slice(start, start + c)
        g = _mx_mm(qx[sl], sx[sl], qw1[e], sw1[e]).bfloat16()
        u = _mx_mm(qx[sl], sx[sl], qw3[e], sw3[e]).bfloat16()
        gs.append(g); us.append(u); hs.append(F.silu(g) * u)
        start += c
    g, u, h = torch.cat(gs), torch.cat(us), torch.cat(hs)
    qh, sh = quant_mxfp8(h)
    ys = []
    start = 0
    for e, c in enumerate(counts.tolist()):
        sl = slice(start, start + c)
        ys.append(_mx_mm(qh[sl], sh[sl], qw2[e], sw2[e]).bfloat16())
        start += c
    return torch.cat(ys), g, u, h


def experts_mxfp8_backward(w1, w2, w3, x, counts, g, u, h, dy):
    """MXFP8 backward matching experts_mxfp8_forward (each grouped GEMM's
    backward as torchao's MX grouped-mm autograd function): dh = dy . w2 with
    dy blocked along D and w2 blocked along D per (expert, h); SwiGLU backward
    in bf16; dx = bf16(dg . w1) + bf16(du . w3) with dg, du and w1, w3 blocked
    along H; dw = per-group products over the expert's tokens, both operands
    blocked along the tokens of the group zero-padded to a multiple of 32."""
    qdy, sdy = quant_mxfp8(dy)
    dgs, dus = [], []
    start = 0
    for e, c in enumerate(counts.tolist()):
        sl = slice(start, start + c)
        qw2t, sw2t = quant_mxfp8(w2[e].t())  # [H, D]
        dh = _mx_mm(qdy[sl], sdy[sl], qw2t, sw2t).bfloat16()
        gg, uu = g[sl], u[sl]
        dsl = dh * uu
        du = dh * F.silu(gg)
        dg = torch.ops.aten.silu_backward(dsl, gg)
        dgs.append(dg); dus.append(du)
        start += c
    dg, du = torch.cat(dgs), torch.cat(dus)
    qdg, sdg = quant_mxfp8(dg)
    qdu, sdu = quant_mxfp8(du)
    dxs, dw1s, dw2s, dw3s = [], [], [], []
    start = 0
    for e, c in enumerate(counts.tolist()):
        sl = slice(start, start + c)
        qw1t, sw1t = quant_mxfp8(w1[e].t())  # [D, H]
        qw3t, sw3t = quant_mxfp8(w3[e].t())
        dxs.append(_mx_mm(qdg[sl], sdg[sl], qw1t, sw1t).bfloat16() + _mx_mm(qdu[sl], sdu[sl], qw3t, sw3t).bfloat16())
        if c == 0:
            dw1s.append(torch.zeros_like(w1[e])); dw3s.append(torch.zeros_like(w3[e])); dw2s.append(torch.zeros_like(w2[e]))
        else:
            def qt(t):
                return quant_mxfp8(_pad_tokens(t[sl].t()))
            (qdgt, sdgt), (qdut, sdut), (qxt, sxt) = qt(dg), qt(du), qt(x)
            (qdyt, sdyt), (qht, sht) = qt(dy), qt(h)
            dw1s.append(_mx_mm(qdgt, sdgt, qxt, sxt).bfloat16())
            dw3s.append(_mx_mm(qdut, sdut, qxt, sxt).bfloat16())
            dw2s.append(_mx_mm(qdyt, sdyt, qht, sht).bfloat16())
        start += c
    return torch.cat(dxs), torch.stack(dw1s), torch.stack(dw2s), torch.stack(dw3s)
