"""Drop-in module API on the CPU: Config dataclasses, state_dict keys and shapes
(torchtitan/models/common/moe.py:73-489, feed_forward.py:34-54), the Kimi
mapping (kimi_linear/model.py:597-707) and the reference's Python-side errors."""

import dataclasses
from types import SimpleNamespace

import pytest
import torch

from torchtitan_amd import FeedForward, GroupedExperts, Linear, MoE, TokenChoiceTopKRouter
from torchtitan_amd.kimi import KimiMoE, init_kimi_moe_weights, kimi_moe_config


def _cfg(d=64, e=8, h=32, hs=48, k=2, coeff=1e-3, groups=None, limited=None, score_func="sigmoid"):
    return MoE.Config(
        num_experts=e,
        experts=GroupedExperts.Config(dim=d, hidden_dim=h, num_experts=e),
        router=TokenChoiceTopKRouter.Config(num_experts=e, gate=Linear.Config(in_features=d, out_features=e),
                                            top_k=k, num_expert_groups=groups, num_limited_groups=limited,
                                            score_func=score_func),
        load_balance_coeff=coeff,
        shared_experts=FeedForward.Config(w1=Linear.Config(in_features=d, out_features=hs),
                                          w2=Linear.Config(in_features=hs, out_features=d),
                                          w3=Linear.Config(in_features=d, out_features=hs)) if hs else None,
    )


def test_state_dict_layout():
    with torch.device("meta"):
        moe = _cfg().build()
    sd = moe.state_dict()
    shapes = {k: tuple(v.shape) for k, v in sd.items()}
    assert shapes == {
        "experts.w1": (8, 32, 64), "experts.w2": (8, 64, 32), "experts.w3": (8, 32, 64),
        "router.gate.weight": (8, 64),
        "shared_experts.w1.weight": (48, 64), "shared_experts.w2.weight": (64, 48),
        "shared_experts.w3.weight": (48, 64),
        "expert_bias": (8,),
    }
    assert sd["expert_bias"].dtype == torch.float32
    # tokens_per_expert is a non-persistent buffer
    assert "tokens_per_expert" in dict(moe.named_buffers()) and "tokens_per_expert" not in sd


def test_no_bias_without_load_balancing_and_no_shared():
    with torch.device("meta"):
        moe = _cfg(coeff=None, hs=0).build()
    assert moe.expert_bias is None and moe.shared_experts is None
    assert set(moe.state_dict()) == {"experts.w1", "experts.w2", "experts.w3", "router.gate.weight"}


def test_config_protocol():
    cfg = _cfg()
    with pytest.raises(TypeError):
        GroupedExperts.Config(8, 4, 2)  # keyword-only
    assert not hasattr(cfg, "__dict__")  # slots
    built = cfg.build()
    assert isinstance(built, MoE) and built.reorderer.top_k == 2
    cfg2 = dataclasses.replace(cfg, score_before_experts=False)
    assert cfg2.build().score_before_experts is False
    assert cfg.to_dict()["router"]["top_k"] == 2


def test_init_states_with_param_init():
    init = {"w1": lambda p: torch.nn.init.constant_(p, 1.0), "w2": lambda p: torch.nn.init.zeros_(p),
            "w3": lambda p: torch.nn.init.constant_(p, 2.0)}
    ex = GroupedExperts.Config(dim=4, hidden_dim=3, num_experts=2, param_init=init).build()
    ex.init_states()
    assert torch.all(ex.w1 == 1) and torch.all(ex.w2 == 0) and torch.all(ex.w3 == 2)
    moe = _cfg(hs=0).build()
    moe._init_self_buffers(buffer_device=torch.device("cpu"))
    assert torch.count_nonzero(moe.expert_bias) == 0 and torch.count_nonzero(moe.tokens_per_expert) == 0


@pytest.mark.parametrize("e,groups,limited,msg", [
    (8, 4, None, "num_limited_groups must be set"),
    (10, 4, 2, "must be divisible"),
    (8, 8, 2, "experts_per_group"),
])
def test_group_config_errors(e, groups, limited, msg):
    r = TokenChoiceTopKRouter.Config(num_experts=e, gate=Linear.Config(in_features=4, out_features=e), top_k=1,
                                     num_expert_groups=groups, num_limited_groups=limited).build()
    with pytest.raises(ValueError, match=msg):
        r(torch.zeros(3, 4))


def test_unknown_score_function():
    r = TokenChoiceTopKRouter.Config(num_experts=4, gate=Linear.Config(in_features=4, out_features=4), top_k=1,
                                     score_func="relu").build()
    with pytest.raises(NotImplementedError):
        r(torch.zeros(3, 4))


def test_feed_forward_is_swiglu():
    ff = FeedForward.Config(w1=Linear.Config(in_features=8, out_features=6),
                            w2=Linear.Config(in_features=6, out_features=8),
                            w3=Linear.Config(in_features=8, out_features=6)).build()
    x = torch.randn(5, 8)
    ref = ff.w2.weight @ (torch.nn.functional.silu(ff.w1.weight @ x.t()) * (ff.w3.weight @ x.t()))
    torch.testing.assert_close(ff(x), ref.t())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_feed_forward_fused_backward_matches_module_autograd(dtype):
    """The shared expert's own backward (dg, du side by side, one GEMM for dW1 and
    dW3) against autograd through the three projections: output, dx and dW2 are
    the same calls and equal bit for bit; dW1 and dW3 are each one fp32-accumulated
    product rounded once, within the bound of such a sum. Tokens are 2-D here: the
    CPU's matmul of a 3-D input is not the folded 2-D product (the GPU's is, and
    the GPU test runs 3-D inputs)."""
    torch.manual_seed(0)
    d, hs, n = 40, 24, 96
    ff = FeedForward.Config(w1=Linear.Config(in_features=d, out_features=hs),
                            w2=Linear.Config(in_features=hs, out_features=d),
                            w3=Linear.Config(in_features=d, out_features=hs)).build().to(dtype)
    x = torch.randn(n, d).to(dtype)
    gy = torch.randn(n, d).to(dtype)
    assert ff._fused_backward_applies(x.clone().requires_grad_(True))
    xa = x.clone().requires_grad_(True)
    out = ff(xa)
    out.backward(gy)
    xb = x.clone().requires_grad_(True)
    w = [lin.weight.detach().clone().requires_grad_(True) for lin in (ff.w1, ff.w2, ff.w3)]
    a1 = torch.nn.functional.linear(xb, w[0])
    a3 = torch.nn.functional.linear(xb, w[2])
    a1.retain_grad()
    a3.retain_grad()
    ref = torch.nn.functional.linear(torch.nn.functional.silu(a1) * a3, w[1])
    ref.backward(gy)
    assert torch.equal(out, ref)
    assert torch.equal(xa.grad, xb.grad)
    assert torch.equal(ff.w2.weight.grad, w[1].grad)
    x2 = x.reshape(n, d).double()
    for lin, a in ((ff.w1, a1), (ff.w3, a3)):
        ga = a.grad.reshape(n, hs).double()
        truth = ga.t() @ x2
        bound = n * 2.0 ** -24 * (ga.abs().t() @ x2.abs())
        ulp = 2.0 ** (torch.floor(torch.log2(truth.abs().clamp_min(2.0 ** -126))) - (23 if dtype == torch.float32 else 7))
        assert ((lin.weight.grad.double() - truth).abs() <= bound + ulp).all()


def test_feed_forward_with_bias_keeps_module_autograd():
    ff = FeedForward.Config(w1=Linear.Config(in_features=8, out_features=6, bias=True),
                            w2=Linear.Config(in_features=6, out_features=8),
                            w3=Linear.Config(in_features=8, out_features=6)).build()
    x = torch.randn(5, 8, requires_grad=True)
    assert not ff._fused_backward_applies(x)
    ff(x).sum().backward()
    assert ff.w1.bias.grad is not None and x.grad is not None


def _ffn(d=64, hs=128):
    return FeedForward.Config(w1=Linear.Config(in_features=d, out_features=hs),
                              w2=Linear.Config(in_features=hs, out_features=d),
                              w3=Linear.Config(in_features=d, out_features=hs)).build()


def test_feed_forward_trains_under_cpu_autocast():
    """Under CPU autocast F.linear returns bf16 activations of fp32 weights: the
    shared expert runs the three modules (autograd), as the reference does, and
    its forward and backward complete with the module path's results."""
    torch.manual_seed(0)
    ff = _ffn()
    x = torch.randn(64, 64, requires_grad=True)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        assert not ff._fused_backward_applies(x)
        out = ff(x)
        ref = ff.w2(torch.nn.functional.silu(ff.w1(x)) * ff.w3(x))
    assert out.dtype == torch.bfloat16 and torch.equal(out, ref)
    out.float().sum().backward()
    assert x.grad is not None and all(lin.weight.grad is not None for lin in (ff.w1, ff.w2, ff.w3))


@pytest.mark.parametrize("where", ["pre", "post", "global"])
def test_feed_forward_hooks_see_the_linear_calls(where):
    """A hook on a projection (or a global module hook) keeps the three module
    calls, so the hook runs; without hooks the fused function reads the weights."""
    ff = _ffn(16, 24)
    x = torch.randn(8, 16, requires_grad=True)
    assert ff._fused_backward_applies(x)
    seen = []
    if where == "pre":
        handle = ff.w1.register_forward_pre_hook(lambda m, a: seen.append(m))
    elif where == "post":
        handle = ff.w2.register_forward_hook(lambda m, a, o: seen.append(m))
    else:
        handle = torch.nn.modules.module.register_module_forward_hook(lambda m, a, o: seen.append(m))
    try:
        assert not ff._fused_backward_applies(x)
        ff(x).sum().backward()
    finally:
        handle.remove()
    assert any(isinstance(m, Linear) for m in seen)
    assert ff._fused_backward_applies(x)


def test_feed_forward_linear_subclass_keeps_its_forward():
    """A Linear subclass with its own forward is called, not bypassed."""

    class Doubled(Linear):
        def forward(self, x):
            return 2 * super().forward(x)

    ff = _ffn(16, 24)
    ff.w2.__class__ = Doubled
    x = torch.randn(8, 16, requires_grad=True)
    assert not ff._fused_backward_applies(x)
    h = torch.nn.functional.silu(ff.w1(x)) * ff.w3(x)
    assert torch.equal(ff(x), 2 * torch.nn.functional.linear(h, ff.w2.weight))


KIMI_48B = SimpleNamespace(
    hidden_size=2304, num_experts=256, num_experts_per_token=8, moe_intermediate_size=1024,
    moe_renormalize=True, moe_router_activation_func="sigmoid", num_shared_experts=1,
    routed_scaling_factor=2.446, num_expert_group=1, topk_group=1,
)


def test_kimi_mapping_and_names():
    cfg = kimi_moe_config(KIMI_48B)
    assert cfg.router.num_expert_groups is None and cfg.router.num_limited_groups is None
    assert cfg.router.route_scale == 2.446 and cfg.router.route_norm and cfg.router.top_k == 8
    assert cfg.shared_experts.w1.out_features == 1024 and cfg.score_before_experts
    grouped = kimi_moe_config(SimpleNamespace(**{**vars(KIMI_48B), "num_expert_group": 8, "topk_group": 4}))
    assert grouped.router.num_expert_groups == 8 and grouped.router.num_limited_groups == 4
    with torch.device("meta"):
        layer = KimiMoE(KIMI_48B)
    names = set(layer.state_dict())
    assert "_moe.experts.w1" in names and "_moe.router.gate.weight" in names and "_moe.expert_bias" in names
    assert tuple(layer._moe.experts.w2.shape) == (256, 2304, 1024)


def test_kimi_init():
    small = SimpleNamespace(**{**vars(KIMI_48B), "hidden_size": 32, "num_experts": 4, "moe_intermediate_size": 16})
    layer = KimiMoE(small)
    layer._moe.expert_bias.fill_(3.0)
    init_kimi_moe_weights(layer, std=0.02)
    assert torch.count_nonzero(layer._moe.expert_bias) == 0
    assert 0.01 < layer._moe.experts.w1.std().item() < 0.03


def _dims(pp=False, cp=False, ep=False):
    return SimpleNamespace(pp_enabled=pp, cp_enabled=cp, ep_enabled=ep)


def test_float8_converter_selects_experts_by_fqn(monkeypatch):
    from torchtitan_amd import quantization as Q

    monkeypatch.setattr(Q, "has_gfx950", lambda: True)
    kw = {"parallel_dims": _dims(), "model_compile_enabled": False}
    model = torch.nn.ModuleDict({"a": _cfg(hs=0).build(), "b": _cfg(hs=0).build()})
    conv_cfg = Q.Float8GroupedMMConverter.Config(fqns=["a.experts"])
    names = conv_cfg.build(**kw).convert(model)
    assert names == ["a.experts"]
    assert model["a"].experts.float8 and not model["b"].experts.float8
    assert set(model["a"].state_dict()) == set(model["b"].state_dict())
    assert Q.find_pad_multiple([conv_cfg]) == 16 and Q.find_pad_multiple([]) is None
    assert Q.Float8GroupedMMConverter.Config(fqns="experts").build(**kw).fqns == ["experts"]


def test_float8_converter_guards_follow_reference():
    """float8.py:238-256: hardware check (ValueError), then no PP and no CP
    (AssertionError with the reference's messages)."""
    from torchtitan_amd import quantization as Q

    cfg = Q.Float8GroupedMMConverter.Config(fqns=["experts"])
    if not Q.has_gfx950():
        with pytest.raises(ValueError, match="only supported on gfx950"):
            cfg.build(parallel_dims=_dims(), model_compile_enabled=True)
    with pytest.raises(TypeError):
        cfg.build()  # parallel_dims and model_compile_enabled are required, as in the reference


def test_float8_converter_rejects_pp_and_cp(monkeypatch):
    from torchtitan_amd import quantization as Q

    monkeypatch.setattr(Q, "has_gfx950", lambda: True)
    cfg = Q.Float8GroupedMMConverter.Config(fqns=["experts"])
    with pytest.raises(AssertionError, match="pipeline parallelism"):
        cfg.build(parallel_dims=_dims(pp=True), model_compile_enabled=True)
    with pytest.raises(AssertionError, match="context parallelism"):
        cfg.build(parallel_dims=_dims(cp=True), model_compile_enabled=True)


def test_mxfp8_converter_selects_experts_by_fqn(monkeypatch):
    from torchtitan_amd import quantization as Q

    monkeypatch.setattr(Q, "has_gfx950", lambda: True)
    kw = {"parallel_dims": _dims(), "model_compile_enabled": True}
    model = torch.nn.ModuleDict({"a": _cfg(hs=0).build(), "b": _cfg(hs=0).build()})
    conv_cfg = Q.MXFP8Converter.Config(fqns="b.experts")
    conv = conv_cfg.build(**kw)
    assert conv.recipe_name == "mxfp8_rceil" and conv.pad_token_groups_for_grouped_mm
    assert not Q.MXFP8Converter.Config(fqns="b.experts").build(
        parallel_dims=_dims(ep=True), model_compile_enabled=True).pad_token_groups_for_grouped_mm
    assert conv.convert(model) == ["b.experts"]
    assert model["b"].experts.mxfp8 and not model["a"].experts.mxfp8
    assert not model["b"].experts.float8
    assert set(model["a"].state_dict()) == set(model["b"].state_dict())
    assert Q.find_pad_multiple([conv_cfg]) == 32
    with pytest.raises(ValueError):
        Q.MXFP8Converter.Config(recipe_name="mxfp8_floor").build(**kw)
    monkeypatch.setattr(Q, "has_gfx950", lambda: False)
    with pytest.raises(AssertionError, match="only supported on gfx950"):
        conv_cfg.build(**kw)


def test_load_balancing_hook_registration_follows_reference_rules():
    """register_moe_load_balancing_hook registers only when the MoE layers have a
    coefficient (optimizer.py:352-362, 439-444); the walk goes layers -> block.moe."""
    from torchtitan_amd.load_balancing import _moe_blocks, register_moe_load_balancing_hook

    class Block(torch.nn.Module):
        def __init__(self, coeff):
            super().__init__()
            self.moe_enabled = True
            self.moe = _cfg(hs=0, coeff=coeff).build()

    class Model(torch.nn.Module):
        def __init__(self, coeff):
            super().__init__()
            self.layers = torch.nn.ModuleDict({"0": Block(coeff), "1": Block(coeff)})

    class Recorder:
        def __init__(self):
            self.hooks = []

        def register_step_pre_hook(self, fn):
            self.hooks.append(fn)

    with_coeff, without = Recorder(), Recorder()
    register_moe_load_balancing_hook(with_coeff, [Model(1e-3)])
    register_moe_load_balancing_hook(without, [Model(None)])
    assert len(with_coeff.hooks) == 1 and without.hooks == []
    assert len(_moe_blocks([Model(1e-3)])) == 2
    # a model without a `layers` dict: every MoE module
    assert len(_moe_blocks([torch.nn.Sequential(_cfg(hs=0).build())])) == 1


def test_gate_gradient_split_is_exact():
    """The gate backward's three bf16 terms add back to the fp32 gradient exactly
    (8 + 8 + 8 significand bits), over twelve decades and both signs; two terms
    would not."""
    from oracle.moe_ref import gate_grad_split3

    g = torch.Generator().manual_seed(3)
    d = torch.randn(512, 64, generator=g) * torch.exp(torch.empty(512, 64).uniform_(-14.0, 14.0, generator=g))
    d[0, :4] = torch.tensor([0.0, -0.0, 1.0 + 2.0 ** -23, -(2.0 - 2.0 ** -23)])
    t = gate_grad_split3(d)
    assert t.dtype == torch.bfloat16 and t.shape == (512, 192)
    hi, mid, lo = (t[:, i * 64:(i + 1) * 64].float() for i in range(3))
    assert torch.equal((hi + mid) + lo, d)
    assert not torch.equal(hi + mid, d)


@pytest.mark.parametrize("halves", [False, True])
def test_gate_dw_reduce_reassembles_the_gradient(halves):
    """dW from the three-term partials: with one-hot token rows every partial sum
    is one exact product, so (hi + mid) + lo of the (half-added) partials is the
    fp32 gradient itself and dW = bf16(d^T x) exactly; dropping a term, or one
    token half, changes the result."""
    from oracle.moe_ref import gate_dw_reduce, gate_grad_split3

    g = torch.Generator().manual_seed(5)
    n, e, dim = 64, 8, 96
    d = torch.randn(n, e, generator=g) * torch.exp(torch.empty(n, e).uniform_(-6.0, 6.0, generator=g))
    x = torch.zeros(n, dim)
    x[torch.arange(n), torch.randperm(dim, generator=g)[:n]] = 1.0  # each token hits its own column
    t = gate_grad_split3(d).float()
    if halves:
        parts = torch.stack([t[: n // 2].t() @ x[: n // 2], t[n // 2:].t() @ x[n // 2:]])
    else:
        parts = t.t() @ x
    want = (d.t() @ x).bfloat16()
    assert torch.equal(gate_dw_reduce(parts, e), want)
    p = parts.clone()
    p[..., 2 * e:, :] = 0.0  # drop lo
    assert not torch.equal(gate_dw_reduce(p, e), want)
    if halves:
        assert not torch.equal(gate_dw_reduce(parts[0], e), want)


def test_routing_counted_once_only_for_the_modules_own_router_and_reorderer():
    """The layer takes the per-expert counts from the reorder alone only when its router and
    reorderer are the module's own types, unhooked, and count_routing_once is set; otherwise
    the router's forward (with its own histogram, moe.py:269-274) is called as in the
    reference, so hooks and subclasses see it."""
    from torchtitan_amd.moe import TokenReorderer

    with torch.device("meta"):
        moe = _cfg().build()
    assert moe._routing_counted_once()
    moe.count_routing_once = False
    assert not moe._routing_counted_once()
    moe.count_routing_once = True
    for mod in (moe.router, moe.reorderer):
        h = mod.register_forward_hook(lambda m, i, o: None)
        assert not moe._routing_counted_once()
        h.remove()
        h = mod.register_forward_pre_hook(lambda m, i: None)
        assert not moe._routing_counted_once()
        h.remove()
    g = torch.nn.modules.module.register_module_forward_hook(lambda m, i, o: None)
    try:
        assert not moe._routing_counted_once()
    finally:
        g.remove()
    assert moe._routing_counted_once()

    class Router(TokenChoiceTopKRouter):
        pass

    class Reorderer(TokenReorderer):
        pass

    with torch.device("meta"):
        sub = _cfg().build()
    sub.router.__class__ = Router
    assert not sub._routing_counted_once()
    sub.router.__class__ = TokenChoiceTopKRouter
    sub.reorderer.__class__ = Reorderer
    assert not sub._routing_counted_once()
