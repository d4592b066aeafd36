"""The drop-in boundary's runtime contract, as torchtitan drives MoE.forward
(torchtitan/models/common/moe.py:380-477):

  * every ``moe_mi355x`` op passes ``torch.library.opcheck`` (schema, fake
    kernel, autograd registration, AOT dispatch with dynamic shapes), the checks
    the reference's own custom op gets from its registration
    (torchtitan/ops/scatter_add.py:10-48);
  * ``router``, ``reorderer`` and ``shared_experts`` compiled as
    apply_compile_sparse does (torchtitan/distributed/compile.py:94-104:
    ``submod.compile(backend, fullgraph=True)``), and the module-level
    ``_run_experts_grouped_mm`` swapped for its fullgraph-compiled self
    (:117-123): forward and backward equal to eager;
  * MoE forward + backward under non-reentrant activation checkpointing, full
    and per-op selective (torchtitan/distributed/activation_checkpoint.py:
    the policy saves matmuls and recomputes the rest): equal to eager, with
    tokens_per_expert counted twice (moe.py:424-426).
"""

import copy
import functools

import pytest
import torch

import torchtitan_amd.moe as moe_module
from tests.conftest import banner
from torchtitan_amd import FeedForward, GroupedExperts, Linear, MoE, TokenChoiceTopKRouter, ops
from torchtitan_amd.feed_forward import swiglu_ffn_backward

pytestmark = pytest.mark.gpu


def _layer(dev, d=256, e=8, k=2, h=256, hs=256, score_func="softmax", score_before=True, seed=0):
    cfg = MoE.Config(
        num_experts=e,
        experts=GroupedExperts.Config(dim=d, hidden_dim=h, num_experts=e),
        router=TokenChoiceTopKRouter.Config(num_experts=e, gate=Linear.Config(in_features=d, out_features=e),
                                            top_k=k, score_func=score_func, route_norm=True, route_scale=2.5),
        score_before_experts=score_before,
        shared_experts=FeedForward.Config(w1=Linear.Config(in_features=d, out_features=hs),
                                          w2=Linear.Config(in_features=hs, out_features=d),
                                          w3=Linear.Config(in_features=d, out_features=hs)) if hs else None,
    )
    moe = cfg.build()
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in moe.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    moe = moe.to(dev)
    for p in moe.parameters():
        p.data = p.data.bfloat16()
    with torch.no_grad():
        moe.expert_bias.copy_(torch.rand(e, generator=gen) * 0.02 - 0.01)
    x = torch.randn(2, 128, d, generator=gen).bfloat16().to(dev)
    g = torch.randn(2, 128, d, generator=gen).bfloat16().to(dev)
    return moe, x, g


def _run(moe, x, g, wrap=None):
    xa = x.clone().requires_grad_(True)
    out = (wrap or moe)(xa)
    out.backward(g)
    grads = {n: p.grad.clone() for n, p in moe.named_parameters()}
    return out.detach(), xa.grad, grads


# ---------------------------------------------------------------------------
# opcheck
# ---------------------------------------------------------------------------


def _distinct_topk(n, e, k, dev, gen):
    return torch.stack([torch.randperm(e, generator=gen)[:k] for _ in range(n)]).to(dev)


def _opcheck_cases(dev):
    gen = torch.Generator().manual_seed(3)
    n, e, k, d, h = 64, 8, 2, 256, 256
    r = n * k

    def bf(*shape, grad=False, scale=1.0):
        return (torch.randn(*shape, generator=gen) * scale).bfloat16().to(dev).requires_grad_(grad)

    def f32(*shape, grad=False):
        return torch.randn(*shape, generator=gen).to(dev).requires_grad_(grad)

    idx = _distinct_topk(n, e, k, dev, gen)
    top = torch.rand(n, k, generator=gen).to(dev)
    scores_sorted, token_idx, counts, offs, slot_pos, tok_pos = ops.reorder(top, idx, e)
    logits = f32(n, e, grad=True)
    _, r_idx, _, r_scores = ops.router(logits.detach(), None, e, k, 1, 0, 0, True, 2.5, False)
    cases = {
        "router": (ops.router, (logits, f32(e), e, k, 1, 0, 0, True, 2.5, False)),
        "router_backward": (ops.router_backward, (f32(n, k), r_scores, r_idx, 1, True, 2.5)),
        "reorder": (ops.reorder, (top.clone().requires_grad_(True), idx, e)),
        "reorder_backward": (ops.reorder_backward, (f32(r), slot_pos)),
        "permute": (ops.permute, (bf(n, d, grad=True), slot_pos, tok_pos, f32(r, grad=True))),
        "permute_backward": (ops.permute_backward, (bf(r, d), bf(n, d), tok_pos, f32(r), True)),
        "combine": (ops.combine, (bf(n, d, grad=True), bf(r, d, grad=True), slot_pos, tok_pos, f32(r, grad=True))),
        "combine_no_shared": (ops.combine, (None, bf(r, d, grad=True), slot_pos, tok_pos, None)),
        "combine_backward": (ops.combine_backward, (bf(n, d), bf(r, d), slot_pos, tok_pos, f32(r))),
        "grouped_swiglu": (ops.grouped_swiglu, (bf(r, d, grad=True), bf(e, h, d, grad=True, scale=0.05),
                                                bf(e, d, h, grad=True, scale=0.05), bf(e, h, d, grad=True, scale=0.05),
                                                counts)),
        "gather_rows": (ops.gather_rows, (bf(r, d, grad=True), torch.randperm(r, generator=gen).to(dev))),
        "scatter_rows": (ops.scatter_rows, (bf(r, d, grad=True), torch.randperm(r, generator=gen).to(dev), r)),
    }
    x = bf(r, d)
    w1, w2, w3 = bf(e, h, d, scale=0.05), bf(e, d, h, scale=0.05), bf(e, h, d, scale=0.05)
    _, gg, uu, hh = ops.grouped_swiglu(x, w1, w2, w3, counts)
    cases["grouped_swiglu_backward"] = (ops.grouped_swiglu_backward, (bf(r, d), x, w1, w2, w3, counts, gg, uu, hh))
    cases["grouped_swiglu_fp8"] = (ops.grouped_swiglu_fp8, (bf(r, d, grad=True), bf(e, h, d, grad=True, scale=0.05),
                                                            bf(e, d, h, grad=True, scale=0.05),
                                                            bf(e, h, d, grad=True, scale=0.05), counts))
    _, g8, u8, h8, *am8 = ops.grouped_swiglu_fp8(x, w1, w2, w3, counts)
    cases["grouped_swiglu_fp8_backward"] = (ops.grouped_swiglu_fp8_backward,
                                            (bf(r, d), x, w1, w2, w3, counts, g8, u8, h8, *am8))
    cases["grouped_swiglu_mxfp8"] = (ops.grouped_swiglu_mxfp8,
                                     (bf(r, d, grad=True), bf(e, h, d, grad=True, scale=0.05),
                                      bf(e, d, h, grad=True, scale=0.05), bf(e, h, d, grad=True, scale=0.05),
                                      counts, True))
    outs = ops.grouped_swiglu_mxfp8(x, w1, w2, w3, counts, True)
    cases["grouped_swiglu_mxfp8_backward"] = (ops.grouped_swiglu_mxfp8_backward,
                                              (bf(r, d), x, w1, w2, w3, counts, *outs[1:]))
    # permute -> MXFP8 experts -> combine as one op (score before the experts)
    def core_args(shared):
        return (bf(n, d, grad=True), bf(n, d, grad=True) if shared else None, token_idx,
                scores_sorted.clone().requires_grad_(True), slot_pos, tok_pos, bf(e, h, d, grad=True, scale=0.05),
                bf(e, d, h, grad=True, scale=0.05), bf(e, h, d, grad=True, scale=0.05), counts)

    cases["moe_core_fp8"] = (ops.moe_core_fp8, core_args(True))
    cases["moe_core_fp8_no_shared"] = (ops.moe_core_fp8, core_args(False))
    core8 = ops.moe_core_fp8(xn_ := bf(n, d), None, token_idx, scores_sorted, slot_pos, tok_pos, w1, w2, w3, counts)
    cases["moe_core_fp8_backward"] = (ops.moe_core_fp8_backward,
                                      (bf(n, d), xn_, token_idx, scores_sorted, tok_pos, w1, w2, w3, counts,
                                       *core8[1:]))
    cases["moe_core_mxfp8"] = (ops.moe_core_mxfp8, core_args(True))
    cases["moe_core_mxfp8_no_shared"] = (ops.moe_core_mxfp8, core_args(False))
    xn = bf(n, d)
    core = ops.moe_core_mxfp8(xn, None, token_idx, scores_sorted, slot_pos, tok_pos, w1, w2, w3, counts)
    cases["moe_core_mxfp8_backward"] = (ops.moe_core_mxfp8_backward,
                                        (bf(n, d), xn, token_idx, scores_sorted, tok_pos, w1, w2, w3, counts,
                                         *core[1:]))
    def f(*shape, grad=False, scale=1.0):
        return (torch.randn(*shape, generator=gen) * scale).to(dev).requires_grad_(grad)

    cases["grouped_swiglu_f32"] = (ops.grouped_swiglu_f32, (f(r, d, grad=True), f(e, h, d, grad=True, scale=0.05),
                                                            f(e, d, h, grad=True, scale=0.05),
                                                            f(e, h, d, grad=True, scale=0.05), counts))
    xf, w1f, w2f, w3f = f(r, d), f(e, h, d, scale=0.05), f(e, d, h, scale=0.05), f(e, h, d, scale=0.05)
    _, gf, uf, hf = ops.grouped_swiglu_f32(xf, w1f, w2f, w3f, counts)
    cases["grouped_swiglu_f32_backward"] = (ops.grouped_swiglu_f32_backward,
                                            (f(r, d), xf, w1f, w2f, w3f, counts, gf, uf, hf))
    m1, m2 = bf(e, 2 * h, d, grad=True, scale=0.05), bf(e, d, h, grad=True, scale=0.05)
    b1, b2 = bf(e, 2 * h, grad=True, scale=0.1), bf(e, d, grad=True, scale=0.1)
    cases["grouped_swiglu_oss"] = (ops.grouped_swiglu_oss, (bf(r, d, grad=True), m1, b1, m2, b2, counts, 7.0))
    _, og, ou, oh = ops.grouped_swiglu_oss(x, m1.detach(), b1.detach(), m2.detach(), b2.detach(), counts, 7.0)
    cases["grouped_swiglu_oss_backward"] = (ops.grouped_swiglu_oss_backward,
                                            (bf(r, d), x, m1.detach(), b1.detach(), m2.detach(), b2.detach(), counts,
                                             og, ou, oh, 7.0))
    # the shared expert's backward (feed_forward.swiglu_ffn_backward) on its forward's intermediates
    hs = 128
    xs, sw1, sw2, sw3 = bf(n, d), bf(hs, d, scale=0.05), bf(d, hs, scale=0.05), bf(hs, d, scale=0.05)
    a1, a3 = torch.nn.functional.linear(xs, sw1), torch.nn.functional.linear(xs, sw3)
    hsw = torch.nn.functional.silu(a1) * a3
    cases["swiglu_ffn_backward"] = (swiglu_ffn_backward, (bf(n, d), xs, sw1, sw2, sw3, a1, a3, hsw,
                                                          True, True, True))
    cases["swiglu_ffn_backward_dw_only"] = (swiglu_ffn_backward, (bf(n, d), xs, sw1, sw2, sw3, a1, a3, hsw,
                                                                  False, True, True))
    cases["swiglu_forward"] = (ops.swiglu_forward, (a1, a3))
    cases["swiglu_backward"] = (ops.swiglu_backward, (bf(n, hs), a1, a3))
    # the gate's backward pieces
    cases["gate_grad_split3"] = (ops.gate_grad_split3, (f32(n, e),))
    cases["gate_dw_reduce"] = (ops.gate_dw_reduce, (f32(2, 3 * e, d), e))
    return cases


OPCHECK_NAMES = ["router", "router_backward", "reorder", "reorder_backward", "permute", "permute_backward",
                 "combine", "combine_no_shared", "combine_backward", "grouped_swiglu", "grouped_swiglu_backward",
                 "grouped_swiglu_f32", "grouped_swiglu_f32_backward",
                 "grouped_swiglu_fp8", "grouped_swiglu_fp8_backward", "grouped_swiglu_mxfp8",
                 "grouped_swiglu_mxfp8_backward", "moe_core_fp8", "moe_core_fp8_no_shared", "moe_core_fp8_backward",
                 "moe_core_mxfp8", "moe_core_mxfp8_no_shared",
                 "moe_core_mxfp8_backward", "grouped_swiglu_oss", "grouped_swiglu_oss_backward",
                 "gather_rows", "scatter_rows", "swiglu_ffn_backward", "swiglu_ffn_backward_dw_only",
                 "swiglu_forward", "swiglu_backward", "gate_grad_split3", "gate_dw_reduce"]


def test_opcheck_covers_every_op():
    ns = torch.ops.moe_mi355x
    registered = {n for n in dir(ns) if isinstance(getattr(ns, n, None), torch._ops.OpOverloadPacket)}
    checked = {n.replace("_no_shared", "").replace("_dw_only", "") for n in OPCHECK_NAMES}
    assert registered <= checked, registered - checked


@pytest.mark.parametrize("name", OPCHECK_NAMES)
def test_opcheck(dev, name):
    banner(f"opcheck {name}")
    op, args = _opcheck_cases(dev)[name]
    torch.library.opcheck(op, args)


# ---------------------------------------------------------------------------
# torch.compile as apply_compile_sparse applies it
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("score_before", [True, False])
def test_compiled_submodules_match_eager(dev, monkeypatch, score_before):
    banner(f"compile router/reorderer/shared_experts + _run_experts_grouped_mm, score_before={score_before}")
    torch._dynamo.reset()
    moe, x, g = _layer(dev, score_before=score_before)
    comp = copy.deepcopy(moe)
    out0, dx0, gr0 = _run(moe, x, g)
    for name in ("router", "reorderer", "shared_experts"):
        getattr(comp, name).compile(backend="aot_eager", fullgraph=True)
    monkeypatch.setattr(moe_module, "_run_experts_grouped_mm",
                        torch.compile(moe_module._run_experts_grouped_mm, backend="aot_eager", fullgraph=True))
    out1, dx1, gr1 = _run(comp, x, g)
    assert torch.equal(comp.tokens_per_expert, moe.tokens_per_expert)
    assert torch.equal(out1, out0)
    for n in gr0:
        assert torch.equal(gr1[n], gr0[n]), n
    # x's gradient sums three branches (gate, routed rows, shared expert) whose
    # order the autograd engine may change once parts of the graph are compiled
    rel = ((dx1.float() - dx0.float()).abs().max() / dx0.float().abs().max()).item()
    print(f"[case] grad_x compiled vs eager: rel {rel:.2e}, identical {torch.equal(dx1, dx0)}", flush=True)
    assert rel <= 1e-2
    torch._dynamo.reset()


# ---------------------------------------------------------------------------
# activation checkpointing
# ---------------------------------------------------------------------------


def _sac_policy():
    """Per-op SAC in the reference's form (activation_checkpoint.py): save the
    matmuls (every second one recomputed) and recompute everything else,
    including the MoE kernels."""
    from torch.utils.checkpoint import CheckpointPolicy

    mm_ops = (torch.ops.aten.mm.default, torch.ops.aten.linear.default, torch.ops.aten.addmm.default)
    meta = {"forward": 0, "recompute": 0}

    def policy(ctx, func, *args, **kwargs):
        if func in mm_ops:
            key = "recompute" if ctx.is_recompute else "forward"
            meta[key] += 1
            return CheckpointPolicy.PREFER_RECOMPUTE if meta[key] % 2 == 0 else CheckpointPolicy.MUST_SAVE
        return CheckpointPolicy.PREFER_RECOMPUTE

    return policy


@pytest.mark.parametrize("mode", ["full", "per_op_sac"])
def test_activation_checkpointing_matches_eager(dev, mode):
    from torch.distributed.algorithms._checkpoint.checkpoint_wrapper import checkpoint_wrapper
    from torch.utils.checkpoint import create_selective_checkpoint_contexts

    banner(f"activation checkpointing {mode}")
    moe, x, g = _layer(dev, seed=5)
    ac = copy.deepcopy(moe)
    out0, dx0, gr0 = _run(moe, x, g)
    if mode == "full":
        wrapped = checkpoint_wrapper(ac)
    else:
        wrapped = checkpoint_wrapper(
            ac, context_fn=functools.partial(create_selective_checkpoint_contexts, _sac_policy()))
    out1, dx1, gr1 = _run(ac, x, g, wrap=wrapped)
    assert torch.equal(out1, out0)
    assert torch.equal(dx1, dx0)
    for n in gr0:
        assert torch.equal(gr1[n], gr0[n]), n
    # the forward runs again in the backward: tokens are counted twice (moe.py:424-426)
    assert torch.equal(ac.tokens_per_expert, 2 * moe.tokens_per_expert)
    assert moe.tokens_per_expert.sum().item() == x.shape[0] * x.shape[1] * 2
