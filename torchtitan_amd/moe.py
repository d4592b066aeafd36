"""Drop-in MoE layer for MI355X: same classes, Config fields, forward signatures
and state_dict layout as torchtitan/models/common/moe.py, with the arithmetic
on hand-written gfx950 kernels (``torchtitan_amd.ops``).

Module map (reference file:line -> here):
  _run_experts_for_loop      moe.py:24-50    -> _run_experts_for_loop
  _run_experts_grouped_mm    moe.py:53-70    -> _run_experts_grouped_mm (ops.grouped_swiglu)
  GroupedExperts             moe.py:73-116   -> GroupedExperts
  TokenChoiceTopKRouter      moe.py:119-276  -> TokenChoiceTopKRouter (gate on torch, rest ops.router)
  TokenReorderer             moe.py:281-332  -> TokenReorderer (ops.reorder)
  MoE                        moe.py:335-489  -> MoE (ops.permute, ops.combine)
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch
from torch import nn

from . import ops
from .configurable import Module, called_plainly
from .feed_forward import FeedForward
from .linear import Linear

__all__ = [
    "GroupedExperts",
    "MoE",
    "ReorderResult",
    "TokenChoiceTopKRouter",
    "TokenReorderer",
    "_run_experts_for_loop",
    "_run_experts_grouped_mm",
    "_run_experts_grouped_mm_fp8",
    "_run_experts_grouped_mm_mxfp8",
]


def _local(t):
    """DTensor -> local shard (moe.py:100-111); plain tensors pass through."""
    to_local = getattr(t, "to_local", None)
    return to_local() if callable(to_local) else t


def _run_experts_for_loop(
    w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor, x: torch.Tensor,
    num_tokens_per_expert: torch.Tensor,
) -> torch.Tensor:
    """Reference readability path (moe.py:24-50): the experts in the input dtype,
    over the first sum(counts) rows, returning those rows.

    fp32 inputs run the fp32 grouped kernels (fp32 products and sums, the SwiGLU
    in fp32, as the reference's fp32 per-expert matmuls); bf16 inputs run the
    bf16 grouped kernels, whose rounding points (each GEMM output, silu and the
    product rounded to bf16) are those of the reference's bf16 matmuls. As in the
    reference, reading sum(counts) synchronises with the host."""
    total = int(num_tokens_per_expert.sum().item())
    xs = x[:total]
    if x.dtype == torch.float32:
        if not (w1.dtype == w2.dtype == w3.dtype == torch.float32):
            raise TypeError(f"expected float32 expert weights for float32 x, got {w1.dtype}, {w2.dtype}, {w3.dtype}")
        y, _, _, _ = ops.grouped_swiglu_f32(xs, w1, w2, w3, num_tokens_per_expert)
        return y
    if x.dtype == torch.bfloat16:
        if not (w1.dtype == w2.dtype == w3.dtype == torch.bfloat16):
            raise TypeError(f"expected bfloat16 expert weights for bfloat16 x, got {w1.dtype}, {w2.dtype}, {w3.dtype}")
        y, _, _, _ = ops.grouped_swiglu(xs, w1, w2, w3, num_tokens_per_expert)
        return y
    raise TypeError(f"the MI355X experts run in float32 or bfloat16, got {x.dtype}")


def _run_experts_grouped_mm(
    w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor, x: torch.Tensor,
    num_tokens_per_expert: torch.Tensor,
) -> torch.Tensor:
    """silu(x w1^T) * (x w3^T) then w2^T per expert segment, bf16 compute with fp32
    accumulation, output cast back to x's dtype (moe.py:53-70)."""
    y, _, _, _ = ops.grouped_swiglu(
        x.bfloat16(), w1.bfloat16(), w2.bfloat16(), w3.bfloat16(), num_tokens_per_expert
    )
    return y.type_as(x)


def _run_experts_grouped_mm_fp8(
    w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor, x: torch.Tensor,
    num_tokens_per_expert: torch.Tensor,
) -> torch.Tensor:
    """The fp8 grouped GEMMs the reference gets from torchao's
    Float8TrainingOpConfig (torchtitan/components/quantization/float8.py:260-288):
    dynamic rowwise e4m3 scaling, fp32 accumulation, bf16 outputs."""
    y, *_ = ops.grouped_swiglu_fp8(
        x.bfloat16(), w1.bfloat16(), w2.bfloat16(), w3.bfloat16(), num_tokens_per_expert
    )
    return y.type_as(x)


def _run_experts_grouped_mm_mxfp8(
    w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor, x: torch.Tensor,
    num_tokens_per_expert: torch.Tensor,
) -> torch.Tensor:
    """The MXFP8 grouped GEMMs the reference gets from torchao's
    MXFP8TrainingOpConfig, recipe "mxfp8_rceil" (torchtitan/components/quantization/mx.py:85-128):
    e4m3 elements with one e8m0 scale per 32 along each contraction, fp32
    accumulation, bf16 outputs."""
    for_backward = torch.is_grad_enabled() and any(t.requires_grad for t in (w1, w2, w3, x))
    y, *_ = ops.grouped_swiglu_mxfp8(
        x.bfloat16(), w1.bfloat16(), w2.bfloat16(), w3.bfloat16(), num_tokens_per_expert, for_backward
    )
    return y.type_as(x)


class GroupedExperts(Module):
    @dataclass(kw_only=True, slots=True)
    class Config(Module.Config):
        dim: int
        hidden_dim: int
        num_experts: int
        use_grouped_mm: bool = True

    def __init__(self, config: Config):
        super().__init__()
        self.num_experts = config.num_experts
        self.w1 = nn.Parameter(torch.empty(config.num_experts, config.hidden_dim, config.dim))
        self.w2 = nn.Parameter(torch.empty(config.num_experts, config.dim, config.hidden_dim))
        self.w3 = nn.Parameter(torch.empty(config.num_experts, config.hidden_dim, config.dim))
        self.use_grouped_mm = config.use_grouped_mm
        # set by quantization.Float8GroupedMMConverter / MXFP8Converter .convert
        self.float8 = False
        self.mxfp8 = False

    def forward(self, x: torch.Tensor, num_tokens_per_expert: torch.Tensor) -> torch.Tensor:
        w1, w2, w3 = _local(self.w1), _local(self.w2), _local(self.w3)
        if self.mxfp8:
            return _run_experts_grouped_mm_mxfp8(w1, w2, w3, x, num_tokens_per_expert)
        if self.float8:
            return _run_experts_grouped_mm_fp8(w1, w2, w3, x, num_tokens_per_expert)
        if self.use_grouped_mm:
            return _run_experts_grouped_mm(w1, w2, w3, x, num_tokens_per_expert)
        return _run_experts_for_loop(w1, w2, w3, x, num_tokens_per_expert)


def _gate_backward_bf16(ctx, grad: torch.Tensor):
    """dx, dW (and the bias gradient) of fp32 logits = x W^T (+ b) for bf16 x and
    W: the fp32 logit gradient d is split exactly into three bf16 terms
    (ops.gate_grad_split3: hi = bf16(d), mid = bf16(d - hi), lo = bf16(d - hi -
    mid), hi + mid + lo == d), and dx, dW are bf16 GEMMs over the 3x longer sum
    -- exact products accumulated in fp32, as the fp32 GEMMs of the autocast
    backward, in another summation order -- rounded to x's and W's dtype once,
    as autocast's casts do."""
    x, w = ctx.saved_tensors
    d3 = ops.gate_grad_split3(grad)
    dx = dw = db = None
    if ctx.needs_input_grad[0]:
        dx = torch.mm(d3, torch.cat([w, w, w], dim=0))  # fp32 accumulation, one rounding to bf16
    if ctx.needs_input_grad[1]:
        e = w.shape[0]
        n = x.shape[0]
        if n >= 8192 and n % 2 == 0:
            # two token halves as a batch of two: the [3E, D] output alone is too few
            # tiles for the chip; the fp32 halves are added before the one rounding
            dw3 = torch.bmm(d3.view(2, n // 2, 3 * e).transpose(1, 2), x.view(2, n // 2, -1),
                            out_dtype=torch.float32)
        else:
            dw3 = torch.mm(d3.t(), x, out_dtype=torch.float32)
        # bf16((hi + mid) + lo) of the (half-summed) fp32 partials, one launch
        dw = ops.gate_dw_reduce(dw3, e)
    if ctx.has_bias and ctx.needs_input_grad[2]:
        db = grad.float().sum(0).to(ctx.b_dtype)
    return dx, dw, db


class _GateRef(torch.autograd.Function):
    """The reference's gate (moe.py:230-232) with a bf16-MFMA backward.

    Forward: F.linear on the fp32 casts of x, W (and b), which is what the
    reference's ``gate(x)`` under ``torch.autocast(dtype=float32)`` runs -- the
    same fp32 GEMM, so the logits, and the routing, are the reference's bits.
    Backward: _gate_backward_bf16, the same exact products as the fp32 backward
    GEMMs, summed in another order, without the fp32 copies of x and W."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None) -> torch.Tensor:
        logits = torch.nn.functional.linear(x.float(), w.float(), b.float() if b is not None else None)
        ctx.save_for_backward(x, w)
        ctx.has_bias = b is not None
        ctx.b_dtype = b.dtype if b is not None else None
        return logits

    backward = staticmethod(_gate_backward_bf16)


class _GateF32(torch.autograd.Function):
    """fp32(x) @ fp32(W)^T (+ fp32(b)) for bf16 x and W, on bf16 GEMMs with fp32
    accumulation and fp32 output.

    A product of two bf16 values is exact in fp32, so the forward equals the fp32
    GEMM of the reference's autocast region (moe.py:230-232) up to summation
    order. The backward is _gate_backward_bf16."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None) -> torch.Tensor:
        logits = torch.mm(x, w.t(), out_dtype=torch.float32)
        if b is not None:
            logits += b.float()
        ctx.save_for_backward(x, w)
        ctx.has_bias = b is not None
        ctx.b_dtype = b.dtype if b is not None else None
        return logits

    backward = staticmethod(_gate_backward_bf16)


def gate_logits_f32(x: torch.Tensor, gate: nn.Linear, bf16_mfma: bool = False) -> torch.Tensor:
    """The router's gate in fp32 (moe.py:230-232).

    The logits are by default those of the reference's own call, ``gate(x)``
    under ``torch.autocast(dtype=float32)``: the same fp32 GEMM, so that top-k
    selection matches it exactly. For bf16 x and W on the GPU (outside an outer
    autocast; E and D multiples of 4) that forward runs in _GateRef, whose backward takes bf16 GEMMs
    over an exact three-term split of the logit gradient instead of fp32 GEMMs;
    anything else runs the autocast region as is.

    ``bf16_mfma=True`` (opt-in) takes _GateF32 for bf16 x and W: the forward
    too on bf16 GEMMs with fp32 accumulation, the same exact products summed in
    another order. A few-ulp logit difference can change a token's expert set
    where its K-th and (K+1)-th biased scores nearly tie."""
    w, b = _local(gate.weight), gate.bias
    b = _local(b) if b is not None else None
    if (x.is_cuda and x.dim() == 2 and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
            and w.shape[0] % 4 == 0 and w.shape[1] % 4 == 0
            and (b is None or b.dtype in (torch.bfloat16, torch.float32))
            and not torch.is_autocast_enabled(x.device.type)):
        fn = _GateF32 if bf16_mfma else _GateRef
        return fn.apply(x.contiguous(), w.contiguous(), b)
    with torch.autocast(device_type=x.device.type, dtype=torch.float32):
        return gate(x)


class TokenChoiceTopKRouter(Module):
    """Token-choice top-K routing with optional group-limited selection."""

    @dataclass(kw_only=True, slots=True)
    class Config(Module.Config):
        num_experts: int
        gate: Linear.Config
        num_expert_groups: int | None = None
        num_limited_groups: int | None = None
        top_k: int = 1
        score_func: Literal["softmax", "sigmoid"] = "sigmoid"
        route_norm: bool = False
        route_scale: float = 1.0
        _debug_force_load_balance: bool = False

    def __init__(self, config: Config):
        super().__init__()
        self.gate = config.gate.build()
        self.num_experts = config.num_experts
        self.num_expert_groups = config.num_expert_groups
        self.num_limited_groups = config.num_limited_groups
        self.top_k = config.top_k
        self.score_func = config.score_func
        self.route_norm = config.route_norm
        self.route_scale = config.route_scale
        self._debug_force_load_balance = config._debug_force_load_balance
        # Opt-in gate on bf16 MFMA with fp32 accumulation (gate_logits_f32); off
        # by default so that the logits, and so the routing, are the reference's.
        self.gate_bf16_mfma = False
        if not 1 <= self.top_k <= ops.MAX_TOP_K:
            raise ValueError(f"top_k ({self.top_k}) must be in [1, {ops.MAX_TOP_K}] for the MI355X router")
        if not 1 <= self.num_experts <= ops.MAX_EXPERTS:
            raise ValueError(
                f"num_experts ({self.num_experts}) must be in [1, {ops.MAX_EXPERTS}] for the MI355X router"
            )

    def _group_config(self) -> tuple[int, int]:
        """Validates the group-limited settings with the reference's errors (moe.py:182-193)."""
        if self.num_expert_groups is None:
            return 0, 0
        if self.num_limited_groups is None:
            raise ValueError("num_limited_groups must be set when num_expert_groups is set")
        if self.num_experts % self.num_expert_groups != 0:
            raise ValueError(
                f"num_experts ({self.num_experts}) must be divisible by num_expert_groups "
                f"({self.num_expert_groups})"
            )
        experts_per_group = self.num_experts // self.num_expert_groups
        if experts_per_group < 2:
            raise ValueError(f"experts_per_group ({experts_per_group}) must be >= 2")
        return self.num_expert_groups, self.num_limited_groups

    def forward(
        self, x: torch.Tensor, expert_bias: torch.Tensor | None = None
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """x [bs*slen, dim] -> (top_scores [N,K] f32, selected_experts_indices [N,K] i64,
        num_tokens_per_expert [E] i64)."""
        return self._route(x, expert_bias, True)

    def _route(self, x: torch.Tensor, expert_bias: torch.Tensor | None, with_counts: bool):
        # fp32 gate logits, as in the reference (moe.py:230-232)
        logits = gate_logits_f32(x, self.gate, self.gate_bf16_mfma)
        if self.score_func not in ops.SCORE_FUNCS:
            raise NotImplementedError(f"Unknown score function {self.score_func}")
        groups, limited = self._group_config()
        top_scores, selected, counts, _scores = ops.router(
            logits, expert_bias, self.num_experts, self.top_k, ops.SCORE_FUNCS[self.score_func],
            groups, limited, bool(self.route_norm), float(self.route_scale),
            bool(self._debug_force_load_balance), with_counts,
        )
        return top_scores, selected, counts


class ReorderResult(tuple):
    """(top_scores_experts_sorted, token_indices_experts_sorted, num_tokens_per_expert),
    unpacked like the reference's 3-tuple, carrying the index layouts the permute
    and combine kernels use: ``offsets`` [E] int32 inclusive cumsum, ``slot_pos``
    [N,K] sorted position of each (token, slot), ``tok_pos`` [N,K] each token's
    sorted positions in ascending order."""

    offsets: torch.Tensor
    slot_pos: torch.Tensor
    tok_pos: torch.Tensor

    def __new__(cls, scores_sorted, token_idx, counts, offsets, slot_pos, tok_pos):
        obj = super().__new__(cls, (scores_sorted, token_idx, counts))
        obj.offsets = offsets
        obj.slot_pos = slot_pos
        obj.tok_pos = tok_pos
        return obj


class TokenReorderer(Module):
    """Reorders (token, slot) pairs into expert-contiguous order (moe.py:281-332)."""

    def __init__(self, *, num_experts: int, top_k: int):
        super().__init__()
        self.num_experts = num_experts
        self.top_k = top_k

    def forward(self, top_scores: torch.Tensor, selected_experts_indices: torch.Tensor) -> ReorderResult:
        return ReorderResult(*ops.reorder(top_scores, selected_experts_indices, self.num_experts))


class MoE(Module):
    @dataclass(kw_only=True, slots=True)
    class Config(Module.Config):
        num_experts: int = 8
        experts: GroupedExperts.Config
        router: TokenChoiceTopKRouter.Config
        score_before_experts: bool = True
        load_balance_coeff: float | None = 1e-3
        shared_experts: FeedForward.Config | None = None

    def __init__(self, config: Config):
        super().__init__()
        num_experts = config.num_experts
        self.experts = config.experts.build()
        self.router = config.router.build()
        self.reorderer = TokenReorderer(num_experts=num_experts, top_k=config.router.top_k)
        self.shared_experts = config.shared_experts.build() if config.shared_experts is not None else None
        self.score_before_experts = config.score_before_experts
        # auxiliary-loss-free load balancing state (moe.py:359-378)
        self.load_balance_coeff = config.load_balance_coeff
        if self.load_balance_coeff is not None:
            assert self.load_balance_coeff > 0.0
            self.register_buffer("expert_bias", torch.zeros(num_experts, dtype=torch.float32), persistent=True)
        else:
            self.expert_bias = None
        self.register_buffer(
            "tokens_per_expert", torch.zeros(num_experts, dtype=torch.float32), persistent=False
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x [bs, slen, dim] -> [bs, slen, dim]."""
        to_local = getattr(x, "to_local", None)
        if callable(to_local):
            from torch.distributed.tensor import Partial

            assert x.device_mesh.ndim == 1, f"Expected 1D mesh, got {x.device_mesh.ndim}D mesh"
            assert x.device_mesh.mesh_dim_names == ("tp",), (
                f"Expected TP mesh, got mesh_dim_names={x.device_mesh.mesh_dim_names}"
            )
            x = x.to_local(grad_placements=(Partial(),))
        bs, slen, dim = x.shape
        x = x.view(-1, dim)

        if self._routing_counted_once():
            # the module's own router and reorderer: the router's histogram (moe.py:269-274)
            # equals the reorderer's (moe.py:312-317) on one GPU, so it is taken once, there
            top_scores, selected_experts_indices, _ = self.router._route(x, self.expert_bias, False)
            layout = self.reorderer(top_scores, selected_experts_indices)
            with torch.no_grad():
                self.tokens_per_expert.add_(layout[2])
        else:
            top_scores, selected_experts_indices, num_tokens_per_expert = self.router(x, self.expert_bias)
            with torch.no_grad():
                self.tokens_per_expert.add_(num_tokens_per_expert)
            layout = self.reorderer(top_scores, selected_experts_indices)
        top_scores_experts_sorted, _token_indices_experts_sorted, num_tokens_per_expert = layout

        core = self._fused_core(x)
        if core is not None:
            # fp8 or MXFP8 experts with the score applied before them: the permute runs
            # inside the experts' token quantizers and the combine's gather inside their
            # backward (ops.moe_core_fp8 / moe_core_mxfp8), with the same results as the
            # three ops
            shared = self.shared_experts(x) if self.shared_experts is not None else None
            experts = self.experts
            out = core(
                x, shared, _token_indices_experts_sorted, top_scores_experts_sorted, layout.slot_pos,
                layout.tok_pos, _local(experts.w1), _local(experts.w2), _local(experts.w3), num_tokens_per_expert,
            )[0]
            return out.reshape(bs, slen, dim)

        # routed_input = x[token_idx] (* score when score_before_experts)
        routed_input = ops.permute(
            x, layout.slot_pos, layout.tok_pos,
            top_scores_experts_sorted if self.score_before_experts else None,
        )
        routed_output = self.experts(routed_input, num_tokens_per_expert)

        out = self.shared_experts(x) if self.shared_experts is not None else None

        # deterministic scatter-add of each token's rows onto the shared output,
        # scaling by the score here when it was not applied before the experts
        out = ops.combine(
            out, routed_output, layout.slot_pos, layout.tok_pos,
            None if self.score_before_experts else top_scores_experts_sorted,
        )
        return out.reshape(bs, slen, dim)

    # set False to run fp8 and MXFP8 experts through the separate permute, experts and
    # combine ops. fp8 experts take the fused op only with fuse_fp8_permute as well:
    # their routed x and dy are each read twice (row and token-transposed
    # quantizations), and gathered twice that measured 0.6 % slower at 32K Kimi
    # tokens than one permuted copy read twice (MXFP8 reads each once, both layouts
    # from one pass, and gains 2 %)
    fuse_permute_into_quantizers = True
    fuse_fp8_permute = False

    # one histogram for the router and the reorderer where both are this module's own
    count_routing_once = True

    def _routing_counted_once(self) -> bool:
        return (self.count_routing_once and type(self.router) is TokenChoiceTopKRouter
                and type(self.reorderer) is TokenReorderer and called_plainly(self.router, self.reorderer))

    def _fused_core(self, x: torch.Tensor):
        """The fused op for this layer's experts, or None where the separate ops run."""
        experts = self.experts
        if not (self.fuse_permute_into_quantizers and type(experts) is GroupedExperts
                and (experts.mxfp8 or experts.float8) and self.score_before_experts and x.is_cuda
                and x.dtype == torch.bfloat16):
            return None
        # the fused op reads the expert weights without calling the experts module:
        # not where hooks on that module expect its call
        if not called_plainly(experts):
            return None
        if not all(_local(w).dtype == torch.bfloat16 for w in (experts.w1, experts.w2, experts.w3)):
            return None
        if experts.mxfp8:
            return ops.moe_core_mxfp8
        # the fp8 row quantizer keeps a row in registers to take the group amax beside it
        if self.fuse_fp8_permute and x.shape[-1] <= ops.AMAX_SIDE_MAX_COLS:
            return ops.moe_core_fp8
        return None

    def _init_self_buffers(self, *, buffer_device: torch.device | None = None) -> None:
        assert isinstance(buffer_device, torch.device)
        with torch.device(buffer_device):
            self.tokens_per_expert = torch.zeros(self.experts.num_experts, dtype=torch.float32)
            if self.load_balance_coeff is not None:
                self.expert_bias = torch.zeros(self.experts.num_experts, dtype=torch.float32)
