"""Pins, on the GPU, the lowering rules the oracle restates for the torch ops the
reference calls, by running those torch ops on the device:
  * torch.topk(sorted=False) selection and slot order (moe.py:199-201, :247-249);
  * torch.sum over a short row (the route_norm denominator, moe.py:264);
  * the deterministic scatter_add (torchtitan/ops/scatter_add.py:10-20);
  * the backward of x[token_idx] (moe.py:445);
  * torch.sigmoid over every fp32 bit pattern, against the router kernel's scores;
and compares the whole drop-in layer with the reference's op sequence run by
torch on the same device (oracle.moe_forward_reference_ops).
"""

import pytest
import torch

from oracle import moe_ref as R
from tests.conftest import banner

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("e", [8, 32, 64, 256, 384, 512])
def test_topk_rule_matches_torch_on_device(dev, e):
    banner(f"pin topk rule E={e}")
    g = torch.Generator().manual_seed(e)
    for k in (1, 2, 4, 8, 16, 32, 64):
        if k > e:
            continue
        for levels in (0, 3, 50):
            v = torch.randn(512, e, generator=g)
            if levels:
                v = torch.round(v * levels) / levels
            _, t_idx = torch.topk(v.to(dev), k, dim=-1, sorted=False)
            o_idx = torch.from_numpy(R.topk_gpu_order(v.numpy(), k))
            assert torch.equal(t_idx.cpu(), o_idx), (e, k, levels)


def test_short_row_sum_order_matches_torch_on_device(dev):
    banner("pin short-row sum order")
    g = torch.Generator().manual_seed(1)
    for k in range(1, 65):
        v = torch.rand(2048, k, generator=g) * torch.exp(torch.randn(2048, k, generator=g) * 4)
        t = v.to(dev).sum(dim=-1).cpu()
        assert torch.equal(t, R.gpu_row_sum(v)), k


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_deterministic_scatter_add_matches_oracle(dev, dtype):
    banner(f"pin deterministic scatter_add {dtype}")
    g = torch.Generator().manual_seed(2)
    n, e, k, d = 1500, 64, 8, 256
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    _, tok, _, _ = R.reorder(torch.rand(n, k, generator=g), idx, e)
    out = torch.randn(n, d, generator=g).to(dtype)
    src = torch.randn(n * k, d, generator=g).to(dtype)
    ref = R._deterministic_scatter_add(out.to(dev), tok.to(dev).reshape(-1, 1).expand(-1, d), src.to(dev))
    assert torch.equal(ref.cpu(), R._Combine.apply(out, tok, src))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_index_backward_matches_oracle(dev, dtype):
    banner(f"pin index backward {dtype}")
    g = torch.Generator().manual_seed(3)
    n, e, k, d = 1500, 64, 8, 256
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    _, tok, _, _ = R.reorder(torch.rand(n, k, generator=g), idx, e)
    grad = torch.randn(n * k, d, generator=g).to(dtype)
    x = torch.zeros(n, d, dtype=dtype, device=dev, requires_grad=True)
    x[tok.to(dev)].backward(grad.to(dev))
    assert torch.equal(x.grad.cpu(), R.index_backward(grad, tok, n))


def test_router_sigmoid_all_fp32_bit_patterns(dev):
    """The router kernel's sigmoid equals torch.sigmoid on the GPU for all 2^32
    inputs (NaNs compared as NaN)."""
    banner("pin sigmoid over all 2^32 fp32 patterns")
    from torchtitan_amd import ops

    e, chunk = 256, 1 << 26
    rows = chunk // e
    mism = 0
    for c in range(1 << 32 >> 26):
        bits = torch.arange(c * chunk, (c + 1) * chunk, dtype=torch.int64, device=dev)
        x = (bits - (1 << 31)).to(torch.int32).view(torch.float32).view(rows, e)
        _, _, _, scores = ops.router(x, None, e, 1, ops.SCORE_FUNCS["sigmoid"], 0, 0, False, 1.0, False)
        ref = torch.sigmoid(x)
        same = (scores == ref) | (torch.isnan(scores) & torch.isnan(ref))
        mism += int((~same).sum())
    assert mism == 0, f"{mism} fp32 inputs where the kernel's sigmoid differs from torch.sigmoid"


LAYER_CASES = {
    # name: (bs, slen, D, E, K, H, Hs, score_func, groups, norm, scale, score_before)
    "kimi_like_small": (2, 512, 512, 256, 8, 256, 256, "sigmoid", None, True, 2.5, True),
    "dsv3_like_small": (1, 512, 512, 64, 8, 256, 512, "sigmoid", (8, 4), True, 2.5, False),
    "softmax_no_shared": (2, 256, 256, 8, 2, 512, 0, "softmax", None, False, 1.0, True),
}


@pytest.mark.parametrize("name", list(LAYER_CASES))
def test_layer_matches_reference_op_sequence_on_device(dev, name):
    """The drop-in MoE (HIP kernels) against the reference's op sequence run by
    torch on the same GPU with the same bf16 parameters: routing bit-exact,
    output and gradients within 1e-2 normwise relative error."""
    bs, slen, d, e, k, h, hs, sf, groups, norm, scale, sb = LAYER_CASES[name]
    banner(f"layer vs reference op sequence {name}")
    from torchtitan_amd import FeedForward, GroupedExperts, Linear, MoE, TokenChoiceTopKRouter

    cfg = MoE.Config(
        num_experts=e,
        experts=GroupedExperts.Config(dim=d, hidden_dim=h, num_experts=e),
        router=TokenChoiceTopKRouter.Config(
            num_experts=e, gate=Linear.Config(in_features=d, out_features=e), top_k=k, score_func=sf,
            route_norm=norm, route_scale=scale, num_expert_groups=groups[0] if groups else None,
            num_limited_groups=groups[1] if groups else None),
        score_before_experts=sb,
        shared_experts=FeedForward.Config(
            w1=Linear.Config(in_features=d, out_features=hs), w2=Linear.Config(in_features=hs, out_features=d),
            w3=Linear.Config(in_features=d, out_features=hs)) if hs else None,
    )
    gen = torch.Generator().manual_seed(21)
    moe = cfg.build()
    with torch.no_grad():
        for p in moe.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    moe = moe.to(dev)
    for p in moe.parameters():
        p.data = p.data.bfloat16()
    with torch.no_grad():
        moe.expert_bias.copy_(torch.rand(e, generator=gen) * 0.02 - 0.01)
    x = torch.randn(bs, slen, d, generator=gen).bfloat16().to(dev)
    gout = torch.randn(bs, slen, d, generator=gen).bfloat16().to(dev)

    xa = x.clone().requires_grad_(True)
    out = moe(xa)
    out.backward(gout)

    sd = moe.state_dict()
    params = {"gate": sd["router.gate.weight"], "w1": sd["experts.w1"], "w2": sd["experts.w2"],
              "w3": sd["experts.w3"], "expert_bias": sd["expert_bias"]}
    if hs:
        params.update(sw1=sd["shared_experts.w1.weight"], sw2=sd["shared_experts.w2.weight"],
                      sw3=sd["shared_experts.w3.weight"])
    params = {n: t.detach().clone().requires_grad_(n != "expert_bias") for n, t in params.items()}
    rc = R.RouterCfg(num_experts=e, top_k=k, score_func=sf, route_norm=norm, route_scale=scale,
                     num_expert_groups=groups[0] if groups else None,
                     num_limited_groups=groups[1] if groups else None)
    mc = R.MoECfg(router=rc, dim=d, hidden_dim=h, score_before_experts=sb, use_grouped_mm=True,
                  has_shared=bool(hs))
    # each side runs its own fp32 gate on the same x (the layer: the reference's
    # autocast call, its default); routing must agree bit for bit
    x2 = x.view(-1, d)
    xb = x.clone().requires_grad_(True)
    try:
        ref = R.moe_forward_reference_ops(params, xb, mc)
    except RuntimeError as err:  # torch._grouped_mm unavailable for this device
        pytest.skip(f"torch._grouped_mm on this device: {err}")
    ref.backward(gout)

    with torch.no_grad():
        top, idx, counts = moe.router(x2, moe.expert_bias)
        with torch.autocast(device_type="cuda", dtype=torch.float32):
            ref_logits = torch.nn.functional.linear(x2, params["gate"].detach())
        t_top, t_idx, t_counts, _ = R.router_forward_torch(ref_logits, params["expert_bias"], rc)
    assert torch.equal(idx, t_idx)
    assert torch.equal(counts, t_counts)
    assert torch.equal(top, t_top)
    errs = {"out": _rel(out, ref), "grad_x": _rel(xa.grad, xb.grad),
            "grad_gate": _rel(moe.router.gate.weight.grad, params["gate"].grad),
            "grad_w1": _rel(moe.experts.w1.grad, params["w1"].grad),
            "grad_w2": _rel(moe.experts.w2.grad, params["w2"].grad),
            "grad_w3": _rel(moe.experts.w3.grad, params["w3"].grad)}
    print(f"[case] {name} rel errors: {errs}", flush=True)
    bad = {n: v for n, v in errs.items() if not v <= 1e-2}
    assert not bad, bad
