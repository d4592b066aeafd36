"""Helpers shared by the GPU layer tests: build the drop-in MoE at a given shape
with device-generated parameters, run it and the reference op sequence
(oracle.moe_forward_reference_ops) on the same GPU, and compare."""

from __future__ import annotations

from dataclasses import dataclass
from types import SimpleNamespace

import torch

from oracle import moe_ref as R

# one GPU: no pipeline, context or expert parallelism
_NO_PARALLEL = SimpleNamespace(pp_enabled=False, cp_enabled=False, ep_enabled=False)


@dataclass
class LayerShape:
    bs: int
    slen: int
    dim: int
    experts: int
    top_k: int
    hidden: int
    shared_hidden: int
    score_func: str = "sigmoid"
    groups: tuple[int, int] | None = None
    route_norm: bool = True
    route_scale: float = 2.5
    score_before: bool = True
    std: float = 0.02
    bias: float = 0.01
    zipf: float | None = None
    fp8: bool = False
    mxfp8: bool = False
    gptoss: bool = False  # gpt-oss experts (GptOssMoE) and a gate with bias
    swiglu_limit: float = 7.0


def build_layer(sh: LayerShape, dev: torch.device, seed: int):
    from torchtitan_amd import FeedForward, GroupedExperts, Linear, MoE, TokenChoiceTopKRouter

    d, e, h, hs = sh.dim, sh.experts, sh.hidden, sh.shared_hidden
    moe_cls = MoE
    extra = {}
    if sh.gptoss:
        from torchtitan_amd.gpt_oss import GptOssMoE

        moe_cls, extra = GptOssMoE, {"swiglu_limit": sh.swiglu_limit}
    cfg = moe_cls.Config(
        num_experts=e,
        experts=GroupedExperts.Config(dim=d, hidden_dim=h, num_experts=e),
        router=TokenChoiceTopKRouter.Config(
            num_experts=e, gate=Linear.Config(in_features=d, out_features=e, bias=sh.gptoss), top_k=sh.top_k,
            score_func=sh.score_func, route_norm=sh.route_norm, route_scale=sh.route_scale,
            num_expert_groups=sh.groups[0] if sh.groups else None,
            num_limited_groups=sh.groups[1] if sh.groups else None),
        score_before_experts=sh.score_before,
        shared_experts=FeedForward.Config(
            w1=Linear.Config(in_features=d, out_features=hs), w2=Linear.Config(in_features=hs, out_features=d),
            w3=Linear.Config(in_features=d, out_features=hs)) if hs else None,
        **extra,
    )
    with torch.device("meta"):
        moe = cfg.build()
    moe = moe.to_empty(device=dev)
    gen = torch.Generator(device=dev).manual_seed(seed)
    with torch.no_grad():
        for p in moe.parameters():
            p.data = torch.empty(p.shape, dtype=torch.bfloat16, device=dev).normal_(0.0, sh.std, generator=gen)
        bias = (torch.rand(e, generator=gen, device=dev) * 2 - 1) * sh.bias
        if sh.zipf:
            ranks = torch.randperm(e, generator=gen, device=dev).float() + 1.0
            bias = bias + 0.25 * ranks.pow(-sh.zipf) - 1.0 * (ranks > e - 20).float()
        moe.expert_bias.copy_(bias)
        moe.tokens_per_expert.zero_()
    if sh.fp8:
        from torchtitan_amd.quantization import Float8GroupedMMConverter

        Float8GroupedMMConverter.Config(fqns=["experts"]).build(
            parallel_dims=_NO_PARALLEL, model_compile_enabled=False).convert(moe)
    if sh.mxfp8:
        from torchtitan_amd.quantization import MXFP8Converter

        MXFP8Converter.Config(fqns=["experts"]).build(
            parallel_dims=_NO_PARALLEL, model_compile_enabled=False).convert(moe)
    x = torch.randn(sh.bs, sh.slen, d, generator=gen, device=dev).bfloat16()
    g = torch.randn(sh.bs, sh.slen, d, generator=gen, device=dev).bfloat16()
    return moe, x, g


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().float(), b.detach().float()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def elem_err(a: torch.Tensor, b: torch.Tensor, floor: float) -> float:
    """The element-wise relative error max |a - b| / (|b| + floor * max |b|): elements
    far below the tensor's scale, where a reordered sum may cancel, are measured
    against `floor` times its largest magnitude instead of their own."""
    a, b = a.detach().float(), b.detach().float()
    fl = floor * b.abs().max().clamp_min(1e-30)
    return ((a - b).abs() / (b.abs() + fl)).max().item()


def compare_with_reference(moe, x: torch.Tensor, g: torch.Tensor, sh: LayerShape) -> dict:
    """Runs both sides forward + backward from the same x and returns
    {name: (rel_err, bit_identical, elem_err at floors 1e-3 and 1e-5)}; asserts that routing (indices, counts, top
    scores) is bit-exact, each side running its own fp32 gate."""
    d = sh.dim
    xa = x.clone().requires_grad_(True)
    out = moe(xa)
    out.backward(g)

    sd = moe.state_dict()
    if sh.gptoss:
        names = {"gate": "router.gate.weight", "gate_bias": "router.gate.bias", "expert_bias": "expert_bias",
                 **{k: f"experts.{k}" for k in ("mlp1_weight", "mlp1_bias", "mlp2_weight", "mlp2_bias")}}
    else:
        names = {"gate": "router.gate.weight", "w1": "experts.w1", "w2": "experts.w2", "w3": "experts.w3",
                 "expert_bias": "expert_bias"}
    if sh.shared_hidden:
        names.update(sw1="shared_experts.w1.weight", sw2="shared_experts.w2.weight",
                     sw3="shared_experts.w3.weight")
    params = {k: sd[v].detach().clone().requires_grad_(k != "expert_bias") for k, v in names.items()}
    rc = R.RouterCfg(num_experts=sh.experts, top_k=sh.top_k, score_func=sh.score_func,
                     route_norm=sh.route_norm, route_scale=sh.route_scale,
                     num_expert_groups=sh.groups[0] if sh.groups else None,
                     num_limited_groups=sh.groups[1] if sh.groups else None)
    mc = R.MoECfg(router=rc, dim=d, hidden_dim=sh.hidden, score_before_experts=sh.score_before,
                  use_grouped_mm=True, has_shared=bool(sh.shared_hidden),
                  expert_kind="gptoss" if sh.gptoss else "swiglu", swiglu_limit=sh.swiglu_limit)
    # each side computes its own gate logits from the same x: the layer with the
    # reference's fp32 autocast call (its default), the oracle with the same call
    # written out; routing must then agree bit for bit
    x2 = x.view(-1, d)
    xb = x.clone().requires_grad_(True)
    aux = {}
    ref = R.moe_forward_reference_ops(params, xb, mc, aux=aux)
    ref.backward(g)

    with torch.no_grad():
        top, idx, counts = moe.router(x2, moe.expert_bias)
        with torch.autocast(device_type=x2.device.type, dtype=torch.float32):
            ref_logits = torch.nn.functional.linear(x2, params["gate"].detach(),
                                                    params["gate_bias"].detach() if "gate_bias" in params else None)
        t_top, t_idx, t_counts, _ = R.router_forward_torch(ref_logits, params["expert_bias"], rc)
    assert torch.equal(idx, t_idx), "selected experts differ from the reference op sequence"
    assert torch.equal(counts, t_counts), "tokens per expert differ"
    assert torch.equal(top, t_top), "top scores differ"
    pairs = {"out": (out, ref), "grad_x": (xa.grad, xb.grad),
             "grad_gate": (moe.router.gate.weight.grad, params["gate"].grad)}
    res_extra = {}
    if sh.gptoss:
        pairs["grad_gate_bias"] = (moe.router.gate.bias.grad, params["gate_bias"].grad)
        for k in ("mlp1_weight", "mlp2_weight"):
            pairs[f"grad_{k}"] = (getattr(moe.experts, k).grad, params[k].grad)
        # bias gradients: the reference sums each expert's rows with bf16 atomics
        # (index_add through repeat_interleave); ours sums in fp32. Both are compared
        # with the exact (fp64) per-expert sums of the reference's own row gradients.
        bounds = torch.cumsum(aux["counts"], 0).tolist()
        def seg_sums(rows):
            rows, out, s0 = rows.double(), [], 0
            for s1 in bounds:
                out.append(rows[s0:s1].sum(0))
                s0 = s1
            return torch.stack(out)
        exact1, exact2 = seg_sums(aux["h1"].grad), seg_sums(aux["y"].grad)
        pairs["grad_mlp1_bias"] = (moe.experts.mlp1_bias.grad, exact1)
        pairs["grad_mlp2_bias"] = (moe.experts.mlp2_bias.grad, exact2)
        res_extra["_ref_bias_grad_err"] = (rel_err(params["mlp1_bias"].grad, exact1),
                                           rel_err(params["mlp2_bias"].grad, exact2))
    else:
        for k in ("w1", "w2", "w3"):
            pairs[f"grad_{k}"] = (getattr(moe.experts, k).grad, params[k].grad)
    res = {k: (rel_err(a, b), bool(torch.equal(a, b)), elem_err(a, b, 1e-3), elem_err(a, b, 1e-5))
           for k, (a, b) in pairs.items()}
    res["_counts"] = counts.cpu()
    res.update(res_extra)
    return res
