"""fp32 experts and the tiny fp32 MoE layer (the reference's CPU-runnable case):
dim 256, 8 routed experts, top-2 softmax router (no route norm, scale 1), no
shared expert, SwiGLU hidden 512, 4096 tokens (2 x 2048), x ~ N(0, 1), fp32
parameters drawn trunc-normal with std 0.02.

  * grouped_swiglu_f32 (the for-loop path's fp32 kernels) forward and backward
    against an fp64 textbook and against the reference's own fp32 for-loop
    (torchtitan/models/common/moe.py:24-50: per-expert torch.matmul in fp32,
    torch's autograd) run on the same GPU: within 2e-5 normwise relative error
    (max |ours - ref| / max |ref|), the spread of two fp32 summation orders;
  * the layer with use_grouped_mm=False against the reference op sequence with
    its fp32 for-loop experts, and with use_grouped_mm=True against the same
    with torch._grouped_mm in bf16 (moe.py:53-70 casts to bf16): routing bit
    exact in both (each side runs its own fp32 gate), outputs and gradients
    within 2e-5 (fp32 experts) and 1e-2 (bf16 experts).
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import moe_ref as R
from tests.conftest import banner
from torchtitan_amd import GroupedExperts, Linear, MoE, TokenChoiceTopKRouter, ops
from torchtitan_amd.moe import _run_experts_for_loop

pytestmark = pytest.mark.gpu

F32_TOL = 2e-5
BF16_TOL = 1e-2


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-300)).item()


def _torch_for_loop(w1, w2, w3, x, counts):
    """moe.py:24-50 as written: per-expert matmuls in x's dtype."""
    outs, s0 = [], 0
    for e, c in enumerate(counts.tolist()):
        xe = x[s0:s0 + c]
        h = F.silu(torch.matmul(xe, w1[e].transpose(-2, -1)))
        h = h * torch.matmul(xe, w3[e].transpose(-2, -1))
        outs.append(torch.matmul(h, w2[e].transpose(-2, -1)))
        s0 += c
    return torch.cat(outs, dim=0)


CASES = {
    "c1_experts": (8, 256, 512, [1100, 950, 1030, 1010, 980, 1040, 990, 1092]),
    "ragged_empty": (6, 192, 320, [0, 77, 1, 0, 300, 63]),
    "one_expert": (1, 128, 128, [513]),
}


@pytest.mark.parametrize("name", list(CASES))
def test_grouped_swiglu_f32_matches_fp32_for_loop(dev, name):
    e, d, h, counts = CASES[name]
    banner(f"fp32 grouped swiglu {name}: E={e} D={d} H={h} counts={counts}")
    g = torch.Generator(device=dev).manual_seed(1)
    r = sum(counts)
    cnt = torch.tensor(counts, device=dev)
    x = torch.randn(r, d, generator=g, device=dev)
    w1, w3 = (torch.randn(e, h, d, generator=g, device=dev) * 0.05 for _ in range(2))
    w2 = torch.randn(e, d, h, generator=g, device=dev) * 0.05
    dy = torch.randn(r, d, generator=g, device=dev)

    ours = [t.clone().requires_grad_(True) for t in (x, w1, w2, w3)]
    y, _, _, _ = ops.grouped_swiglu_f32(ours[0], ours[1], ours[2], ours[3], cnt)
    y.backward(dy)

    ref = [t.clone().requires_grad_(True) for t in (x, w1, w2, w3)]
    yr = _torch_for_loop(ref[1], ref[2], ref[3], ref[0], cnt)
    yr.backward(dy)

    f64 = [t.double().requires_grad_(True) for t in (x, w1, w2, w3)]
    y64 = _torch_for_loop(f64[1], f64[2], f64[3], f64[0], cnt.cpu())
    y64.backward(dy.double())

    names = ("x", "w1", "w2", "w3")
    errs = {"out": (_rel(y, y64), _rel(yr, y64), _rel(y, yr))}
    for n, a, b, c in zip(names, ours, ref, f64):
        errs[f"grad_{n}"] = (_rel(a.grad, c.grad), _rel(b.grad, c.grad), _rel(a.grad, b.grad))
    print(f"[case] {name} (ours vs fp64, torch fp32 vs fp64, ours vs torch fp32): "
          + ", ".join(f"{k} {v[0]:.1e}/{v[1]:.1e}/{v[2]:.1e}" for k, v in errs.items()), flush=True)
    for k, (ours_err, torch_err, vs_torch) in errs.items():
        assert ours_err <= F32_TOL and vs_torch <= F32_TOL, (k, ours_err, vs_torch)
    for n, a in zip(names[1:], ours[1:]):
        for ei, c in enumerate(counts):
            if c == 0:
                assert torch.count_nonzero(a.grad[ei]) == 0, f"grad_{n} of empty expert {ei}"


def test_for_loop_keeps_dtype_and_rows(dev):
    """fp32 stays fp32 (no bf16 rounding anywhere), bf16 runs the bf16 kernels,
    and, as the reference, only the first sum(counts) rows come back."""
    g = torch.Generator(device=dev).manual_seed(2)
    e, d, h = 4, 128, 192
    counts = torch.tensor([10, 0, 20, 7], device=dev)
    x = torch.randn(40, d, generator=g, device=dev)
    w1, w3 = (torch.randn(e, h, d, generator=g, device=dev) * 0.05 for _ in range(2))
    w2 = torch.randn(e, d, h, generator=g, device=dev) * 0.05
    y = _run_experts_for_loop(w1, w2, w3, x, counts)
    assert y.shape == (37, d) and y.dtype == torch.float32
    ref = _torch_for_loop(w1.double(), w2.double(), w3.double(), x[:37].double(), counts.cpu())
    assert _rel(y, ref) <= F32_TOL
    assert _rel(y, y.bfloat16().float()) > 0  # not bf16-rounded
    yb = _run_experts_for_loop(w1.bfloat16(), w2.bfloat16(), w3.bfloat16(), x.bfloat16(), counts)
    rb = _torch_for_loop(w1.bfloat16(), w2.bfloat16(), w3.bfloat16(), x[:37].bfloat16(), counts.cpu())
    assert yb.dtype == torch.bfloat16 and yb.shape == (37, d) and _rel(yb, rb) <= BF16_TOL
    with pytest.raises(TypeError):
        _run_experts_for_loop(w1.bfloat16(), w2, w3, x, counts)


def _c1_layer(dev, use_grouped_mm: bool, seed: int = 0):
    d, e, k, h = 256, 8, 2, 512
    cfg = MoE.Config(
        num_experts=e,
        experts=GroupedExperts.Config(dim=d, hidden_dim=h, num_experts=e, use_grouped_mm=use_grouped_mm),
        router=TokenChoiceTopKRouter.Config(num_experts=e, gate=Linear.Config(in_features=d, out_features=e),
                                            top_k=k, score_func="softmax", route_norm=False, route_scale=1.0),
        score_before_experts=True,
        shared_experts=None,
    )
    moe = cfg.build()
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in moe.parameters():
            p.copy_(torch.nn.init.trunc_normal_(torch.empty(p.shape), std=0.02, a=-0.04, b=0.04, generator=gen))
    moe = moe.to(dev)
    x = torch.randn(2, 2048, d, generator=gen).to(dev)
    gout = torch.randn(2, 2048, d, generator=gen).to(dev)
    return moe, x, gout


@pytest.mark.parametrize("use_grouped_mm", [False, True])
def test_c1_layer_matches_reference_op_sequence(dev, use_grouped_mm):
    banner(f"c1 fp32 layer, use_grouped_mm={use_grouped_mm}")
    moe, x, gout = _c1_layer(dev, use_grouped_mm)
    d = x.shape[-1]
    xa = x.clone().requires_grad_(True)
    out = moe(xa)
    out.backward(gout)
    assert out.dtype == torch.float32

    sd = moe.state_dict()
    params = {"gate": sd["router.gate.weight"], "w1": sd["experts.w1"], "w2": sd["experts.w2"],
              "w3": sd["experts.w3"], "expert_bias": sd["expert_bias"]}
    params = {n: t.detach().clone().requires_grad_(n != "expert_bias") for n, t in params.items()}
    rc = R.RouterCfg(num_experts=8, top_k=2, score_func="softmax", route_norm=False, route_scale=1.0)
    mc = R.MoECfg(router=rc, dim=d, hidden_dim=512, score_before_experts=True, use_grouped_mm=use_grouped_mm,
                  has_shared=False)
    xb = x.clone().requires_grad_(True)
    ref = R.moe_forward_reference_ops(params, xb, mc)
    ref.backward(gout)

    x2 = x.view(-1, d)
    with torch.no_grad():
        top, idx, counts = moe.router(x2, moe.expert_bias)
        with torch.autocast(device_type="cuda", dtype=torch.float32):
            logits = F.linear(x2, params["gate"].detach())
        t_top, t_idx, t_counts, _ = R.router_forward_torch(logits, params["expert_bias"], rc)
    assert torch.equal(idx, t_idx) and torch.equal(counts, t_counts) and torch.equal(top, t_top)

    errs = {"out": _rel(out, ref), "grad_x": _rel(xa.grad, xb.grad),
            "grad_gate": _rel(moe.router.gate.weight.grad, params["gate"].grad)}
    for n in ("w1", "w2", "w3"):
        errs[f"grad_{n}"] = _rel(getattr(moe.experts, n).grad, params[n].grad)
    tol = BF16_TOL if use_grouped_mm else F32_TOL
    print(f"[case] c1 use_grouped_mm={use_grouped_mm}: counts {counts.tolist()}; "
          + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()) + f" (bound {tol:g})", flush=True)
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, bad
