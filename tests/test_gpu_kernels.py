"""GPU parity of the MI355X kernels against the oracle (oracle/moe_ref.py).

Bars:
  * routing indices, token counts, permutation, permute and combine: bit-exact;
  * bf16 GEMM outputs and gradients: normwise max relative error
    max|ours - ref| / max|ref| <= 1e-2 against the fp32-accumulated reference.
"""

import numpy as np
import pytest
import torch

from oracle import moe_ref as R
from tests.conftest import banner

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


def ops():
    from torchtitan_amd import ops as _ops

    return _ops


ROUTER_CASES = {
    # name: (N, E, K, score_func, groups, limited, norm, scale, bias, force_lb, tie_levels)
    "tiny_softmax_e8_k2": (4096, 8, 2, "softmax", None, None, False, 1.0, False, False, 0),
    "kimi_sigmoid_bias_e256_k8": (4096, 256, 8, "sigmoid", None, None, True, 2.5, True, False, 0),
    "dsv3_group_limited": (2048, 256, 8, "sigmoid", 8, 4, True, 2.5, True, False, 0),
    "softmax_e96_k6": (1024, 96, 6, "softmax", None, None, True, 1.0, False, False, 0),
    "ties_sigmoid_e64_k4": (2048, 64, 4, "sigmoid", None, None, False, 1.0, False, False, 5),
    "ties_group_e32_g4": (1024, 32, 4, "sigmoid", 4, 2, True, 1.0, False, False, 3),
    "force_load_balance": (1000, 16, 3, "sigmoid", None, None, True, 1.0, False, True, 0),
    # eight experts per lane, K past a wave's eighth, ties and a bias
    "ties_sigmoid_e512_k16": (1024, 512, 16, "sigmoid", None, None, True, 1.0, True, False, 4),
    # E not a multiple of 64 with five experts per lane
    "softmax_e320_k10": (1024, 320, 10, "softmax", None, None, True, 2.0, False, False, 0),
    "ties_group_e512_g16_k12": (1024, 512, 12, "sigmoid", 16, 5, True, 1.0, True, False, 6),
    # two experts per lane with ties and a bias; four per lane with E not a multiple of 64
    "ties_sigmoid_bias_e128_k8": (2048, 128, 8, "sigmoid", None, None, True, 2.5, True, False, 4),
    "ties_softmax_e200_k7": (2048, 200, 7, "softmax", None, None, False, 1.0, False, False, 3),
}


def _router_inputs(n, e, tie_levels, bias, seed):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(n, e, generator=g)
    if tie_levels:
        logits = torch.round(logits * tie_levels) / tie_levels  # many exact ties
    b = (torch.rand(e, generator=g) * 0.02 - 0.01) if bias else None
    if tie_levels and bias:
        b = torch.round(b * 100) / 100
    return logits, b


@pytest.mark.parametrize("name", list(ROUTER_CASES))
def test_router_bit_exact(dev, name):
    n, e, k, sf, groups, limited, norm, scale, bias, flb, ties = ROUTER_CASES[name]
    banner(f"router {name}")
    logits, b = _router_inputs(n, e, ties, bias, seed=1234)
    cfg = R.RouterCfg(num_experts=e, top_k=k, score_func=sf, num_expert_groups=groups,
                      num_limited_groups=limited, route_norm=norm, route_scale=scale,
                      force_load_balance=flb)
    o = ops()
    top, idx, counts, scores = o.router(
        logits.to(dev), b.to(dev) if b is not None else None, e, k, o.SCORE_FUNCS[sf],
        groups or 0, limited or 0, norm, scale, flb,
    )
    torch.cuda.synchronize()
    # 1. score function: bit-identical to torch's on the device
    ref_scores = R.score_fn(logits.to(dev), sf)
    assert torch.equal(scores, ref_scores), "score function differs from torch on the GPU"
    # 2. selection, slot order, gathered/normalised scores: bit-exact vs the oracle
    o_top, o_idx, o_counts, _ = R.router_forward(None, b, cfg, scores=scores.cpu())
    assert torch.equal(idx.cpu(), o_idx), "selected experts differ from the oracle"
    assert torch.equal(counts.cpu(), o_counts)
    assert torch.equal(top.cpu(), o_top), "top scores differ from the oracle"
    # 3. and identical to the reference op sequence run by torch on the GPU
    t_top, t_idx, t_counts, _ = R.router_forward_torch(logits.to(dev), b.to(dev) if b is not None else None, cfg)
    assert torch.equal(idx, t_idx)
    assert torch.equal(counts, t_counts)
    assert torch.equal(top, t_top)
    # 4. without the histogram: the same selection and scores, no counts
    top2, idx2, counts2, scores2 = o.router(
        logits.to(dev), b.to(dev) if b is not None else None, e, k, o.SCORE_FUNCS[sf],
        groups or 0, limited or 0, norm, scale, flb, False,
    )
    assert torch.equal(top2, top) and torch.equal(idx2, idx) and torch.equal(scores2, scores)
    assert counts2.numel() == 0


@pytest.mark.parametrize("name", ["kimi_sigmoid_bias_e256_k8", "tiny_softmax_e8_k2", "dsv3_group_limited"])
def test_router_backward(dev, name):
    n, e, k, sf, groups, limited, norm, scale, bias, flb, ties = ROUTER_CASES[name]
    banner(f"router backward {name}")
    logits, b = _router_inputs(n, e, ties, bias, seed=99)
    g = torch.randn(n, k, generator=torch.Generator().manual_seed(5))
    o = ops()
    lg = logits.to(dev).requires_grad_(True)
    top, idx, counts, scores = o.router(lg, b.to(dev) if b is not None else None, e, k,
                                        o.SCORE_FUNCS[sf], groups or 0, limited or 0, norm, scale, flb)
    (top * g.to(dev)).sum().backward()
    # oracle gradient: same selection, autograd through the restated ops in fp64
    cfg = R.RouterCfg(num_experts=e, top_k=k, score_func=sf, num_expert_groups=groups,
                      num_limited_groups=limited, route_norm=norm, route_scale=scale)
    l64 = logits.double().requires_grad_(True)
    s64 = R.score_fn(l64, sf)
    ts = s64.gather(1, idx.cpu())
    if norm:
        ts = ts / (ts.sum(-1, keepdim=True) + 1e-20)
    ts = ts * scale
    (ts * g.double()).sum().backward()
    assert rel_err(lg.grad, l64.grad) < 1e-5


# (tokens, experts, top-k): the scan folded into the scatter (per-block counts of at most
# 32768 words, E a multiple of 4), and the separate scan kernel (E = 62; 157 x 512 words)
REORDER_CASES = {"fused_e64": (5000, 64, 6), "kimi_fused_e256": (16384, 256, 8),
                 "scan_e62": (5000, 62, 6), "scan_e512": (40000, 512, 8)}


@pytest.mark.parametrize("name", list(REORDER_CASES))
def test_reorder_exact(dev, name):
    banner(f"reorder {name}")
    n, e, k = REORDER_CASES[name]
    logits, _ = _router_inputs(n, e, 0, False, seed=7)
    o = ops()
    top, idx, _, _ = o.router(logits.to(dev), None, e, k, 1, 0, 0, False, 1.0, False)
    ss, tok, counts, offs, slot_pos, tok_pos = o.reorder(top, idx, e)
    torch.cuda.synchronize()
    r_ss, r_tok, r_counts, r_perm = R.reorder(top.cpu(), idx.cpu(), e)
    assert torch.equal(tok.cpu(), r_tok)
    assert torch.equal(ss.cpu(), r_ss)
    assert torch.equal(counts.cpu(), r_counts)
    assert torch.equal(offs.cpu().long(), torch.cumsum(r_counts, 0))
    # slot_pos is the inverse of the stable argsort, tok_pos its per-token sorted rows
    inv = torch.empty_like(r_perm)
    inv[r_perm] = torch.arange(r_perm.numel())
    assert torch.equal(slot_pos.cpu().long().view(-1), inv)
    assert torch.equal(tok_pos.cpu().long(), torch.sort(inv.view(n, k), dim=1).values)
    # torch's own stable argsort on the device agrees
    assert torch.equal(tok, torch.argsort(idx.view(-1), stable=True) // k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("score_before", [True, False])
def test_permute_combine_exact(dev, dtype, score_before):
    banner(f"permute/combine dtype={dtype} score_before={score_before}")
    n, e, k, d = 3000, 32, 4, 512
    gen = torch.Generator().manual_seed(11)
    logits = torch.randn(n, e, generator=gen)
    x = torch.randn(n, d, generator=gen).to(dtype)
    shared = torch.randn(n, d, generator=gen).to(dtype)
    routed = torch.randn(n * k, d, generator=gen).to(dtype)
    gout = torch.randn(n, d, generator=gen).to(dtype)
    o = ops()
    top, idx, _, _ = o.router(logits.to(dev), None, e, k, 1, 0, 0, True, 2.0, False)
    ss, tok, counts, offs, slot_pos, tok_pos = o.reorder(top, idx, e)
    xs = x.to(dev).requires_grad_(True)
    sc = ss.detach().clone().requires_grad_(True)
    # permute
    ri = o.permute(xs, slot_pos, tok_pos, sc if score_before else None)
    ref = x[tok.cpu()]
    if score_before:
        ref = (ref.float() * ss.cpu().reshape(-1, 1)).to(dtype)
    assert torch.equal(ri.detach().cpu(), ref)
    # combine (forward) vs the oracle's deterministic scatter-add restatement
    rs = routed.to(dev).requires_grad_(True)
    sh = shared.to(dev).requires_grad_(True)
    out = o.combine(sh, rs, slot_pos, tok_pos, None if score_before else sc)
    src = routed if score_before else (routed.float() * ss.cpu().reshape(-1, 1)).to(dtype)
    r_out = R._Combine.apply(shared, tok.cpu(), src)
    assert torch.equal(out.detach().cpu(), r_out)
    # backward of the combine and of the permute
    out.backward(gout.to(dev))
    assert torch.equal(sh.grad.cpu(), gout)
    gr_ref = gout[tok.cpu()]
    if not score_before:
        gr_ref = (gr_ref.float() * ss.cpu().reshape(-1, 1)).to(dtype)
    assert torch.equal(rs.grad.cpu(), gr_ref)
    gri = torch.randn(n * k, d, generator=gen).to(dtype)
    ri.backward(gri.to(dev))
    g_in = gri if not score_before else (gri.float() * ss.cpu().reshape(-1, 1)).to(dtype)
    assert torch.equal(xs.grad.cpu(), R.index_backward(g_in, tok.cpu(), n))
    # score gradients (fp32 dot products over D; order differs from torch's reduction)
    if score_before:
        ds_ref = (gri.double() * x[tok.cpu()].double()).sum(1)
    else:
        ds_ref = (gout[tok.cpu()].double() * routed.double()).sum(1)
    assert rel_err(sc.grad, ds_ref) < 1e-5


def _gemm_inputs(e, d, h, counts, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    r = int(sum(counts))
    x = torch.randn(r, d, generator=g).bfloat16()
    w1 = (torch.randn(e, h, d, generator=g) * std).bfloat16()
    w2 = (torch.randn(e, d, h, generator=g) * std).bfloat16()
    w3 = (torch.randn(e, h, d, generator=g) * std).bfloat16()
    dy = torch.randn(r, d, generator=g).bfloat16()
    return x, w1, w2, w3, dy, torch.tensor(counts, dtype=torch.int64)


GEMM_CASES = {
    "uniform_e8": (8, 256, 512, [130, 128, 127, 1, 255, 256, 257, 100]),
    "empty_and_skewed": (8, 512, 256, [0, 700, 0, 3, 0, 0, 129, 0]),
    "single_expert": (1, 256, 256, [333]),
    # D, H multiples of 64 but not of the tile widths: partial last n- and m-tiles
    "tails_d320_h192": (6, 320, 192, [100, 0, 257, 31, 64, 200]),
    "tails_d2880_h2880": (3, 2880, 2880, [300, 0, 77]),
    # D a multiple of 384: the dx kernel's 128 x 384 tile, w1 half parked in registers
    "dx_d768_h320": (5, 768, 320, [90, 0, 300, 129, 17]),
    # tall experts (875 rows each on average): gate_up and down on their 256 x 256 tiles with
    # 64-wide k-steps, partial last n-tiles (2H = 384, D = 320) and an empty expert
    "tall_tails_d320_h192": (4, 320, 192, [1000, 0, 1500, 1000]),
}


@pytest.mark.parametrize("name", list(GEMM_CASES))
def test_grouped_swiglu_fwd_bwd(dev, name):
    e, d, h, counts = GEMM_CASES[name]
    banner(f"grouped swiglu {name}")
    x, w1, w2, w3, dy, cnt = _gemm_inputs(e, d, h, counts, seed=3)
    o = ops()
    xs, w1s, w2s, w3s = (t.to(dev).requires_grad_(True) for t in (x, w1, w2, w3))
    y, g, u, hh = o.grouped_swiglu(xs, w1s, w2s, w3s, cnt.to(dev))
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    # fp32 reference from the same bf16 inputs, with the reference's bf16 roundings
    xr, w1r, w2r, w3r = (t.float().requires_grad_(True) for t in (x, w1, w2, w3))
    ys, gs, us, hs = [], [], [], []
    start = 0
    for ei, c in enumerate(counts):
        xe = xr[start : start + c]
        ge = xe @ w1r[ei].t()
        ue = xe @ w3r[ei].t()
        he = torch.nn.functional.silu(ge) * ue
        ys.append(he @ w2r[ei].t())
        gs.append(ge); us.append(ue); hs.append(he)
        start += c
    yr = torch.cat(ys)
    yr.backward(dy.float())
    assert rel_err(y, yr) < BF16_TOL
    assert rel_err(g, torch.cat(gs)) < BF16_TOL
    assert rel_err(u, torch.cat(us)) < BF16_TOL
    assert rel_err(hh, torch.cat(hs)) < BF16_TOL
    assert rel_err(xs.grad, xr.grad) < BF16_TOL
    for ours, ref, nm in ((w1s.grad, w1r.grad, "w1"), (w2s.grad, w2r.grad, "w2"), (w3s.grad, w3r.grad, "w3")):
        assert rel_err(ours, ref) < BF16_TOL, nm
        for ei, c in enumerate(counts):
            if c == 0:
                assert torch.count_nonzero(ours[ei]).item() == 0, f"{nm}[{ei}] of an empty expert"
    # forward also matches the oracle's bf16 grouped-mm restatement
    assert rel_err(y, R.experts_grouped_mm(w1, w2, w3, x, cnt)) < BF16_TOL


def test_grouped_swiglu_deterministic(dev):
    banner("grouped swiglu run-to-run")
    e, d, h, counts = GEMM_CASES["uniform_e8"]
    x, w1, w2, w3, dy, cnt = _gemm_inputs(e, d, h, counts, seed=4)
    o = ops()
    outs = []
    for _ in range(2):
        xs, w1s, w2s, w3s = (t.to(dev).requires_grad_(True) for t in (x, w1, w2, w3))
        y, *_ = o.grouped_swiglu(xs, w1s, w2s, w3s, cnt.to(dev))
        y.backward(dy.to(dev))
        outs.append([y.detach(), xs.grad, w1s.grad, w2s.grad, w3s.grad])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


# torch._grouped_mm and its autograd on the same GPU (the reference's own call,
# moe.py:53-70). Both accumulate in fp32 and round to bf16 at the same points;
# at the benchmark shapes every element is identical, at other shapes torch's
# GEMM may order the k sum differently, which flips a rounding in a few elements:
# at these shapes at most 1e-4 of the elements may differ (where torch splits a
# long k sum, as at D >= 4096 with a few hundred rows per expert, a few tenths of
# a percent do), by at most one bf16 ulp of the
# tensor's largest magnitude (dx sums two bf16 halves, so a flip in one half
# can exceed the ulp of the element itself). Shapes cover
# the dx kernel's register park (D % 384 == 0) and its in-memory park (D % 512 == 0).
BIT_CASES = {  # experts, D, H, seed, expert rows drawn from [lo, hi)
    "d768_h512": (16, 768, 512, 3, 0, 400),
    "d1024_h512": (8, 1024, 512, 5, 0, 400),
    # tall experts: the forward on its 256 x 256 tiles
    "tall_d768_h512": (6, 768, 512, 7, 700, 1400),
    # H = 2048: dw13's 16 m-tiles per expert take the blocked tile order
    "dw13_blocked_d512_h2048": (4, 512, 2048, 9, 100, 500),
}


@pytest.mark.parametrize("name", list(BIT_CASES))
def test_grouped_swiglu_vs_torch_grouped_mm(dev, name):
    e, d, h, seed, lo, hi = BIT_CASES[name]
    banner(f"grouped swiglu vs torch._grouped_mm {name}")
    g = torch.Generator().manual_seed(seed)
    counts = torch.randint(lo, hi, (e,), generator=g)
    counts[1] = 0
    x, w1, w2, w3, dy, cnt = _gemm_inputs(e, d, h, counts.tolist(), seed=seed)
    o = ops()
    xs, w1s, w2s, w3s = (t.to(dev).requires_grad_(True) for t in (x, w1, w2, w3))
    y, gg, uu, hh = o.grouped_swiglu(xs, w1s, w2s, w3s, cnt.to(dev))
    y.backward(dy.to(dev))
    xr, w1r, w2r, w3r = (t.to(dev).requires_grad_(True) for t in (x, w1, w2, w3))
    offs = torch.cumsum(cnt.to(dev), 0, dtype=torch.int32)
    gr = torch._grouped_mm(xr, w1r.transpose(-2, -1), offs=offs)
    ur = torch._grouped_mm(xr, w3r.transpose(-2, -1), offs=offs)
    hr = torch.nn.functional.silu(gr) * ur
    yr = torch._grouped_mm(hr, w2r.transpose(-2, -1), offs=offs)
    yr.backward(dy.to(dev))
    torch.cuda.synchronize()
    pairs = {"y": (y, yr), "g": (gg, gr), "u": (uu, ur), "h": (hh, hr), "dx": (xs.grad, xr.grad),
             "dw1": (w1s.grad, w1r.grad), "dw2": (w2s.grad, w2r.grad), "dw3": (w3s.grad, w3r.grad)}
    diff = {k: (a != b).sum().item() for k, (a, b) in pairs.items()}
    print(f"[case] {name}: counts {counts.tolist()}, differing elements {diff}", flush=True)
    for k, (a, b) in pairs.items():
        assert diff[k] <= 1e-4 * a.numel(), (k, diff[k], a.numel())
        assert rel_err(a, b) <= 2.0 ** -7, (k, rel_err(a, b))



# Seeded random shapes beyond the bit-exact cases: tall experts (the 256 x 256 forward
# tiles), long contractions (D >= 4096: the 128 x 256 64-wide forward tile), ragged
# and empty experts. Where torch's grouped mm orders a long k sum differently a few
# tenths of a percent of the elements are one rounding apart (seen up to 0.41 %), so
# the bound is the rounding itself: relative difference <= 2^-7 of the tensor maximum,
# at most 1 % of the elements differing, and against an fp64 restatement our g is no
# further off than torch's.
RANDOM_SHAPE_CASES = {  # experts, D, H, expert rows drawn from [lo, hi), seed
    "tall_e5_d1088_h448": (5, 1088, 448, 300, 1400, 467317),
    "tall_e7_d1152_h256": (7, 1152, 256, 300, 1400, 702866),
    "long_e4_d4160_h128": (4, 4160, 128, 0, 400, 21363),
    "long_e6_d4352_h256": (6, 4352, 256, 0, 400, 633321),
    "small_e11_d256_h448": (11, 256, 448, 0, 300, 971512),
}


@pytest.mark.parametrize("name", list(RANDOM_SHAPE_CASES))
def test_grouped_swiglu_random_shapes(dev, name):
    e, d, h, lo, hi, seed = RANDOM_SHAPE_CASES[name]
    banner(f"grouped swiglu random shape {name}")
    g = torch.Generator().manual_seed(seed)
    counts = torch.randint(lo, hi, (e,), generator=g)
    if e > 2:
        counts[e // 2] = 0
    x, w1, w2, w3, dy, cnt = _gemm_inputs(e, d, h, counts.tolist(), seed=seed)
    o = ops()
    xs, w1s, w2s, w3s = (t.to(dev).requires_grad_(True) for t in (x, w1, w2, w3))
    y, gg, uu, hh = o.grouped_swiglu(xs, w1s, w2s, w3s, cnt.to(dev))
    y.backward(dy.to(dev))
    xr, w1r, w2r, w3r = (t.to(dev).requires_grad_(True) for t in (x, w1, w2, w3))
    offs = torch.cumsum(cnt.to(dev), 0, dtype=torch.int32)
    gr = torch._grouped_mm(xr, w1r.transpose(-2, -1), offs=offs)
    ur = torch._grouped_mm(xr, w3r.transpose(-2, -1), offs=offs)
    hr = torch.nn.functional.silu(gr) * ur
    yr = torch._grouped_mm(hr, w2r.transpose(-2, -1), offs=offs)
    yr.backward(dy.to(dev))
    torch.cuda.synchronize()
    pairs = {"y": (y, yr), "g": (gg, gr), "u": (uu, ur), "h": (hh, hr), "dx": (xs.grad, xr.grad),
             "dw1": (w1s.grad, w1r.grad), "dw2": (w2s.grad, w2r.grad), "dw3": (w3s.grad, w3r.grad)}
    diff = {k: (a != b).sum().item() for k, (a, b) in pairs.items()}
    print(f"[case] {name}: counts {counts.tolist()}, differing elements {diff}", flush=True)
    for k, (a, b) in pairs.items():
        assert diff[k] <= 1e-2 * a.numel(), (k, diff[k], a.numel())
        assert rel_err(a, b) <= 2.0 ** -7, (k, rel_err(a, b))
    g64, s = [], 0
    for ei, c in enumerate(counts.tolist()):
        g64.append(x[s:s + c].double() @ w1[ei].double().t())
        s += c
    g64 = torch.cat(g64)
    err_ours = (gg.detach().cpu().double() - g64).abs().max().item()
    err_torch = (gr.detach().cpu().double() - g64).abs().max().item()
    assert err_ours <= err_torch * 1.01 + 1e-12, (err_ours, err_torch)


def test_layer_counts_routing_once(dev):
    """With its own router and reorderer the layer takes the per-expert counts from the
    reorder's histogram only (moe.py:312-317; the router's, moe.py:269-274, is the same
    on one GPU): output, gradients and tokens_per_expert equal the two-histogram path's,
    and a hook on the router brings the router's own call back."""
    from tests.layer_util import LayerShape, build_layer

    banner("layer routing counted once vs twice")
    sh = LayerShape(bs=2, slen=512, dim=512, experts=16, top_k=4, hidden=256, shared_hidden=256)
    moe, x, gy = build_layer(sh, dev, seed=5)

    def run(once):
        moe.count_routing_once = once
        moe.zero_grad(set_to_none=True)
        moe.tokens_per_expert.zero_()
        xx = x.clone().requires_grad_(True)
        assert moe._routing_counted_once() == once
        out = moe(xx)
        out.backward(gy)
        torch.cuda.synchronize()
        return out.detach(), xx.grad, moe.tokens_per_expert.clone(), {n: p.grad.clone() for n, p in moe.named_parameters()}

    a, b = run(False), run(True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])
    assert a[2].sum().item() == sh.bs * sh.slen * sh.top_k
    for n in a[3]:
        assert torch.equal(a[3][n], b[3][n]), n
    seen = []
    handle = moe.router.register_forward_hook(lambda m, i, o: seen.append(o[2].clone()))
    try:
        assert not moe._routing_counted_once()
        moe.tokens_per_expert.zero_()
        moe(x)
        torch.cuda.synchronize()
        assert len(seen) == 1 and torch.equal(seen[0].float(), moe.tokens_per_expert)
    finally:
        handle.remove()


# Every bf16 bit pattern, in-range values (where the epilogues use the reciprocal
# form: -80 <= g <= 3.38e38) first so that those pieces take that form, the rest
# (below -80, infinities, NaNs) after.
def _bf16_patterns_split():
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    v = bits.view(torch.bfloat16)
    f = v.float()
    fast = (f >= -80.0) & (f <= 3.38e38)
    return v[fast], v[~fast]


def test_swiglu_pointwise_every_bf16(dev):
    """The SwiGLU epilogues' silu and sigmoid (moe.py:62-67 through torch's silu
    and its backward) for all 65536 bf16 inputs, in fp32 before any rounding,
    equal torch's F.silu and torch.sigmoid of the same values on the device: the
    reciprocal-and-correction form is the IEEE quotient wherever it is used."""
    banner("swiglu pointwise, every bf16 input")
    from torchtitan_amd import _lib

    fast, rest = _bf16_patterns_split()
    assert fast.numel() % 2 == 0
    for order in ("split", "natural"):
        g = torch.cat([fast, rest]) if order == "split" else torch.cat([fast, rest]).view(torch.int16).sort().values.view(torch.bfloat16)
        g = g.to(dev)
        silu = torch.empty(g.numel(), dtype=torch.float32, device=dev)
        sig = torch.empty_like(silu)
        _lib.call("moe_swiglu_pointwise_f32", g.data_ptr(), silu.data_ptr(), sig.data_ptr(), g.numel(),
                  _lib.stream_of(g))
        ref_silu = torch.nn.functional.silu(g.float())
        ref_sig = torch.sigmoid(g.float())
        for name, a, b in (("silu", silu, ref_silu), ("sigmoid", sig, ref_sig)):
            same = (a.view(torch.int32) == b.view(torch.int32)) | (torch.isnan(a) & torch.isnan(b))
            bad = (~same).nonzero().flatten()[:8].cpu()
            assert bad.numel() == 0, (order, name, [(float(g[i].float()), float(a[i]), float(b[i])) for i in bad])


def _fill_rows(vals, rows, cols):
    """vals repeated to fill [rows, cols] row by row."""
    n = rows * cols
    rep = (n + vals.numel() - 1) // vals.numel()
    return vals.repeat(rep)[:n].view(rows, cols)


@pytest.mark.parametrize("rows", [320, 1280])
def test_gate_up_epilogue_every_bf16(dev, rows):
    """gate_up with one-hot token rows, so that g = x.w1^T is w1's entries exactly
    and covers every finite bf16 value: h equals torch's silu(g) * u bit for bit,
    in the pieces that take the reciprocal form (rows 0-207 of each 320) and in
    the ones that divide (rows 208-319)."""
    banner(f"gate_up epilogue, every finite bf16 g, {rows} rows")
    from torchtitan_amd import _lib

    d, h = 320, 256
    fast, rest = _bf16_patterns_split()
    rest = rest[torch.isfinite(rest.float())]
    gt = torch.cat([_fill_rows(fast, 208, h), _fill_rows(rest, 112, h)])  # [320, H]: g of token row r
    gen = torch.Generator().manual_seed(11)
    w1 = gt.t().contiguous().view(1, h, d)
    w3 = (torch.randn(1, h, d, generator=gen) * 2).bfloat16()
    x = torch.zeros(rows, d, dtype=torch.bfloat16)
    x[torch.arange(rows), torch.arange(rows) % d] = 1.0
    x, w1, w3 = x.to(dev), w1.to(dev), w3.to(dev)
    counts = torch.tensor([rows], dtype=torch.int64, device=dev)
    g = torch.empty(rows, h, dtype=torch.bfloat16, device=dev)
    u, hh = torch.empty_like(g), torch.empty_like(g)
    _lib.call("moe_grouped_gemm_gate_up", x.data_ptr(), w1.data_ptr(), w3.data_ptr(), counts.data_ptr(), rows, 1,
              d, h, g.data_ptr(), u.data_ptr(), hh.data_ptr(), _lib.stream_of(x))
    # g is w1's entry itself, except that -0 comes out +0 and the MFMA may flush
    # subnormal operands
    gt_rows = gt.to(dev)[torch.arange(rows, device=dev) % d]
    tiny = gt_rows.float().abs() < 2.0 ** -126
    assert bool(((g.view(torch.int16) == gt_rows.view(torch.int16)) | tiny).all())
    ref = torch.nn.functional.silu(g) * u
    same = (hh.view(torch.int16) == ref.view(torch.int16)) | (torch.isnan(hh) & torch.isnan(ref))
    assert bool(same.all()), int((~same).sum())


@pytest.mark.parametrize("rows", [320, 1280])
def test_dgu_epilogue_every_bf16(dev, rows):
    """bwd_dgu with one-hot output-gradient rows, so that dh = dy.w2 is w2's entries
    exactly, on g covering every bf16 value (NaNs and infinities included): dg and
    du equal torch's autograd of silu(g) * u bit for bit (NaNs as NaNs)."""
    banner(f"dgu epilogue, every bf16 g, {rows} rows")
    from torchtitan_amd import _lib

    d, h = 320, 256
    fast, rest = _bf16_patterns_split()
    gt = torch.cat([_fill_rows(fast, 208, h), _fill_rows(rest, 112, h)])
    gen = torch.Generator().manual_seed(12)
    g = gt[torch.arange(rows) % d].contiguous()
    u = (torch.randn(rows, h, generator=gen) * 2).bfloat16()
    w2 = (torch.randn(1, d, h, generator=gen) * 2).bfloat16()
    dy = torch.zeros(rows, d, dtype=torch.bfloat16)
    dy[torch.arange(rows), torch.arange(rows) % d] = 1.0
    g, u, w2, dy = g.to(dev), u.to(dev), w2.to(dev), dy.to(dev)
    counts = torch.tensor([rows], dtype=torch.int64, device=dev)
    dgu = torch.empty(rows, 2 * h, dtype=torch.bfloat16, device=dev)
    _lib.call("moe_grouped_gemm_bwd_dgu", dy.data_ptr(), w2.data_ptr(), g.data_ptr(), u.data_ptr(),
              counts.data_ptr(), rows, 1, d, h, dgu.data_ptr(), _lib.stream_of(dy))
    dh = w2[0][torch.arange(rows, device=dev) % d]
    gr, ur = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
    (torch.nn.functional.silu(gr) * ur).backward(dh)
    for name, a, b in (("dg", dgu[:, :h], gr.grad), ("du", dgu[:, h:], ur.grad)):
        same = (a.view(torch.int16) == b.view(torch.int16)) | (torch.isnan(a) & torch.isnan(b))
        assert bool(same.all()), (name, int((~same).sum()))
