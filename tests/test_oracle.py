"""Pins the oracle (oracle/moe_ref.py) on the CPU.

What fixes each function, independently of the formula being checked:
  * generate_permute_indices: the reference's own known-answer vectors
    (tests/golden/ep_permute_kats.json, from tests/unit_tests/test_expert_parallel.py);
  * radix_key, topk_gpu_order, node_limited_choice, select_experts: brute force
    over tiny inputs and, where there are no ties, torch's CPU topk run through the
    reference's op sequence (router_forward_torch);
  * gpu_row_sum: exact on integer-valued floats, and the explicit trees for n=6, 8;
  * reorder: brute-force stable sort by (expert, flat position) and the EP=1
    identity of generate_permute_indices;
  * _Combine / index_backward: sequential loops, ATen's CPU scatter_add (which
    adds rows into the destination in index order, in its dtype) and the
    autograd of x[token_idx] in fp32;
  * experts_grouped_mm / experts_for_loop: torch._grouped_mm on the CPU (the
    reference's third-party call) and a float64 textbook loop;
  * router gradients: float64 finite differences;
  * moe_forward: the reference op sequence (moe_forward_reference_ops) on the CPU;
  * expert_bias_update: closed forms on hand-worked loads (balanced, one hot
    expert, ties with the mean, the recomputation halving);
  * quant_mxfp8 / _mx_mm: an independent bit-level derivation of the RCEIL
    exponent (biased exponent of amax / 448, +1 for a non-zero mantissa),
    hand-worked blocks, values on the e4m3 grid that must round-trip exactly,
    power-of-two equivariance, the e4m3 rounding bound, and exact GEMMs of
    grid values whose blocks carry different scales;
  * experts_fp8_forward / experts_fp8_backward: operands on the e4m3 grid with
    power-of-two scales along the recipe's axes, where every GEMM must equal
    the fp64 product rounded once (the SwiGLU gradient from torch's autograd),
    two planted mistakes (weights scaled along the contraction; transposed
    operands scaled along the other axis) that these pins must catch, and a
    bound of 0.1 against an fp64 autograd reference.
The GPU-lowering rules the oracle states (top-k tie order, deterministic
scatter-add order, index-backward rounding, short-row sum order) are pinned
against torch on the device in tests/test_gpu_oracle_pins.py.
"""

import itertools
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_ref as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------------------
# EP permute indices: the reference's known-answer vectors
# ---------------------------------------------------------------------------


def _kats():
    with open(os.path.join(GOLDEN, "ep_permute_kats.json")) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _kats(), ids=lambda c: c["name"])
def test_generate_permute_indices_known_answers(case):
    idx, ntok = R.generate_permute_indices(case["tokens_per_expert_group"], case["experts_per_rank"],
                                           case["num_ranks"])
    total = sum(case["tokens_per_expert_group"])
    assert idx.shape == (total,)
    assert sorted(idx.tolist()) == list(range(total))
    if case["expected_indices"] is not None:
        assert idx.tolist() == case["expected_indices"]
    if case["expected_num_tokens"] is not None:
        assert ntok.tolist() == case["expected_num_tokens"]


def test_permute_indices_planted_mistake_is_caught():
    """A transposed (rank-major) output would pass the permutation check but not
    the known answers."""
    case = _kats()[0]
    wrong = np.arange(sum(case["tokens_per_expert_group"]))
    assert wrong.tolist() != case["expected_indices"]


# ---------------------------------------------------------------------------
# selection rules
# ---------------------------------------------------------------------------


def _total_order(v: float):
    """Textbook total order of floats used by a radix select: NaN above all,
    -0 below +0."""
    if np.isnan(v):
        return (2, 0.0, 0)
    return (1, v, 0 if np.signbit(v) else 1)


def test_radix_key_is_the_total_order():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(200).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4e38, -3.4e38], dtype=np.float32),
    ])
    keys = R.radix_key(vals)
    for i in range(len(vals)):
        for j in range(0, len(vals), 7):
            a, b = _total_order(float(vals[i])), _total_order(float(vals[j]))
            assert (keys[i] < keys[j]) == (a < b)
            assert (keys[i] == keys[j]) == (a == b or (np.isnan(vals[i]) and np.isnan(vals[j])))


def _brute_topk(row, k):
    keys = [_total_order(float(v)) for v in row]
    order = sorted(range(len(row)), key=lambda i: (tuple(-x if isinstance(x, float) else -x for x in keys[i]), i))
    chosen = order[:k]
    kth = keys[chosen[-1]]
    above = sorted(i for i in chosen if keys[i] > kth)
    ties = sorted(i for i in chosen if keys[i] == kth)
    return above + ties


def test_topk_gpu_order_brute_force_with_ties():
    rng = np.random.default_rng(1)
    levels = np.array([-1.0, 0.0, -0.0, 0.5, 0.5, 2.0], dtype=np.float32)
    for e in range(1, 7):
        for k in range(1, e + 1):
            vals = rng.choice(levels, size=(40, e)).astype(np.float32)
            got = R.topk_gpu_order(vals, k)
            for r in range(vals.shape[0]):
                assert got[r].tolist() == _brute_topk(vals[r], k), (e, k, vals[r])


def test_topk_set_matches_torch_without_ties():
    g = torch.Generator().manual_seed(2)
    v = torch.randn(500, 64, generator=g)
    for k in (1, 4, 8):
        got = R.topk_gpu_order(v.numpy(), k)
        _, ref = torch.topk(v, k, dim=-1, sorted=False)
        assert torch.equal(torch.sort(torch.from_numpy(got), 1).values, torch.sort(ref, 1).values)


def _brute_node_limited(row, n_groups, n_limited):
    e = len(row)
    epg = e // n_groups
    gs = []
    for g in range(n_groups):
        grp = sorted(row[g * epg:(g + 1) * epg], key=_total_order, reverse=True)
        gs.append(np.float32(grp[0]) + np.float32(grp[1]))
    keep = set(_brute_topk(np.array(gs, dtype=np.float32), n_limited))
    return np.array([row[i] if (i // epg) in keep else -np.inf for i in range(e)], dtype=np.float32)


def test_node_limited_choice_brute_force():
    rng = np.random.default_rng(3)
    for (e, g, gk) in ((8, 4, 2), (12, 3, 1), (16, 8, 4), (6, 3, 3)):
        vals = np.round(rng.standard_normal((30, e)) * 2) / 2  # ties
        vals = vals.astype(np.float32)
        got = R.node_limited_choice(vals, g, gk)
        for r in range(vals.shape[0]):
            np.testing.assert_array_equal(got[r], _brute_node_limited(vals[r], g, gk))


@pytest.mark.parametrize("sf,groups,norm,bias", [
    ("sigmoid", None, True, True), ("softmax", None, False, False), ("sigmoid", (8, 4), True, True),
    ("softmax", (4, 2), True, False),
])
def test_router_matches_reference_op_sequence_on_cpu(sf, groups, norm, bias):
    """No exact ties in random fp32 logits: the reference op sequence run by torch
    on the CPU selects the same sets; scores agree to rounding."""
    g = torch.Generator().manual_seed(4)
    n, e, k = 300, 64, 6
    logits = torch.randn(n, e, generator=g)
    b = torch.rand(e, generator=g) * 0.02 - 0.01 if bias else None
    cfg = R.RouterCfg(num_experts=e, top_k=k, score_func=sf, route_norm=norm, route_scale=2.5,
                      num_expert_groups=groups[0] if groups else None,
                      num_limited_groups=groups[1] if groups else None)
    top, idx, counts, scores = R.router_forward(logits, b, cfg)
    t_top, t_idx, t_counts, t_scores = R.router_forward_torch(logits, b, cfg)
    assert torch.equal(scores, t_scores)
    si, order = torch.sort(idx, 1)
    ti, torder = torch.sort(t_idx, 1)
    assert torch.equal(si, ti)
    torch.testing.assert_close(top.gather(1, order), t_top.gather(1, torder), rtol=1e-6, atol=0)
    assert torch.equal(counts, t_counts)
    assert int(counts.sum()) == n * k


def test_force_load_balance_round_robin():
    cfg = R.RouterCfg(num_experts=5, top_k=3, force_load_balance=True)
    idx = R.select_experts(np.zeros((7, 5), np.float32), None, cfg)
    assert idx.reshape(-1).tolist() == [i % 5 for i in range(21)]


def test_score_fn_rejects_unknown():
    with pytest.raises(NotImplementedError):
        R.score_fn(torch.zeros(2, 2), "relu")


# ---------------------------------------------------------------------------
# short-row sum order
# ---------------------------------------------------------------------------


def test_gpu_row_sum_exact_on_integers_and_trees():
    v = torch.arange(1, 65, dtype=torch.float32).reshape(1, 64)
    for n in range(1, 65):
        assert R.gpu_row_sum(v[:, :n]).item() == n * (n + 1) / 2
    x = torch.randn(5, 8, dtype=torch.float32)
    tree8 = ((x[:, 0] + x[:, 1]) + (x[:, 2] + x[:, 3])) + ((x[:, 4] + x[:, 5]) + (x[:, 6] + x[:, 7]))
    assert torch.equal(R.gpu_row_sum(x), tree8)
    y = x[:, :6]
    tree6 = ((y[:, 0] + y[:, 4]) + (y[:, 1] + y[:, 5])) + (y[:, 2] + y[:, 3])
    assert torch.equal(R.gpu_row_sum(y), tree6)


# ---------------------------------------------------------------------------
# reorder
# ---------------------------------------------------------------------------


def test_reorder_is_stable_sort_by_expert_then_position():
    g = torch.Generator().manual_seed(5)
    n, e, k = 200, 16, 4
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    top = torch.rand(n, k, generator=g)
    ss, tok, counts, perm = R.reorder(top, idx, e)
    flat = idx.reshape(-1).tolist()
    brute = sorted(range(n * k), key=lambda p: (flat[p], p))
    assert perm.tolist() == brute
    assert tok.tolist() == [p // k for p in brute]
    assert torch.equal(ss, top.reshape(-1)[torch.tensor(brute)])
    assert counts.tolist() == [flat.count(i) for i in range(e)]
    # token ids ascend inside each expert segment, and a token appears once per expert
    start = 0
    for c in counts.tolist():
        seg = tok[start:start + c].tolist()
        assert seg == sorted(seg) and len(set(seg)) == len(seg)
        start += c


def test_reorder_is_slot_order_invariant():
    g = torch.Generator().manual_seed(6)
    n, e, k = 100, 12, 3
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    top = torch.rand(n, k, generator=g)
    shuffle = torch.stack([torch.randperm(k, generator=g) for _ in range(n)])
    a = R.reorder(top, idx, e)
    b = R.reorder(top.gather(1, shuffle), idx.gather(1, shuffle), e)
    for x, y in zip(a[:3], b[:3]):
        assert torch.equal(x, y)


def test_ep1_permute_indices_are_identity():
    idx, ntok = R.generate_permute_indices([5, 0, 3, 2], 4, 1)
    assert idx.tolist() == list(range(10)) and ntok.tolist() == [5, 0, 3, 2]


# ---------------------------------------------------------------------------
# combine and index backward
# ---------------------------------------------------------------------------


def _seq_combine(out, token_idx, src):
    acc = out.clone()
    for p, t in enumerate(token_idx.tolist()):
        acc[t] = (acc[t].float() + src[p].float()).to(out.dtype)
    return acc


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_combine_matches_sequential_loop(dtype):
    g = torch.Generator().manual_seed(7)
    n, e, k, d = 64, 8, 3, 16
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    _, tok, _, _ = R.reorder(torch.rand(n, k, generator=g), idx, e)
    out = torch.randn(n, d, generator=g).to(dtype)
    src = torch.randn(n * k, d, generator=g).to(dtype)
    got = R._Combine.apply(out, tok, src)
    assert torch.equal(got, _seq_combine(out, tok, src))
    if dtype == torch.float32:
        # ATen's CPU scatter_add adds the source rows into the destination in
        # index order in fp32: the same sequence of fp32 additions. (In bf16 the
        # CPU kernel accumulates in fp32 and rounds once, unlike the GPU's sorted
        # index_put, so only fp32 pins the order here.)
        ref = R._deterministic_scatter_add(out, tok.reshape(-1, 1).expand(-1, d), src)
        assert torch.equal(got, ref)


def test_index_backward_matches_loop_with_rounding():
    g = torch.Generator().manual_seed(8)
    n, d = 40, 8
    tok = torch.sort(torch.randint(0, n, (120,), generator=g)).values
    grad = torch.randn(120, d, generator=g).bfloat16()
    got = R.index_backward(grad, tok, n)
    ref = torch.zeros(n, d, dtype=torch.bfloat16)
    for p, t in enumerate(tok.tolist()):
        ref[t] = (ref[t].float() + grad[p].float()).bfloat16()
    assert torch.equal(got, ref)
    # fp32: the same sums as autograd of x[token_idx]
    x = torch.zeros(n, d, requires_grad=True)
    x[tok].backward(grad.float())
    torch.testing.assert_close(R.index_backward(grad.float(), tok, n), x.grad, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# experts
# ---------------------------------------------------------------------------


def _expert_inputs(e, d, h, counts, seed):
    g = torch.Generator().manual_seed(seed)
    r = sum(counts)
    return (torch.randn(r, d, generator=g), torch.randn(e, h, d, generator=g) * 0.05,
            torch.randn(e, d, h, generator=g) * 0.05, torch.randn(e, h, d, generator=g) * 0.05,
            torch.tensor(counts))


def test_experts_grouped_mm_matches_torch_grouped_mm():
    x, w1, w2, w3, c = _expert_inputs(4, 32, 48, [5, 0, 17, 9], 9)
    got = R.experts_grouped_mm(w1, w2, w3, x.bfloat16(), c)
    offs = torch.cumsum(c, 0, dtype=torch.int32)
    xb = x.bfloat16()
    hh = F.silu(torch._grouped_mm(xb, w1.bfloat16().transpose(-2, -1), offs=offs))
    hh = hh * torch._grouped_mm(xb, w3.bfloat16().transpose(-2, -1), offs=offs)
    ref = torch._grouped_mm(hh, w2.bfloat16().transpose(-2, -1), offs=offs)
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-2, atol=2e-2)


def test_experts_for_loop_matches_float64_textbook():
    x, w1, w2, w3, c = _expert_inputs(3, 16, 24, [4, 7, 2], 10)
    got = R.experts_for_loop(w1, w2, w3, x, c)
    rows = []
    start = 0
    for e, n in enumerate(c.tolist()):
        for r in range(start, start + n):
            xr = x[r].double()
            gg = w1[e].double() @ xr
            uu = w3[e].double() @ xr
            hh = gg / (1 + torch.exp(-gg)) * uu
            rows.append(w2[e].double() @ hh)
        start += n
    torch.testing.assert_close(got.double(), torch.stack(rows), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# router gradient
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("sf,norm", [("sigmoid", True), ("softmax", False), ("softmax", True)])
def test_router_gradient_finite_differences(sf, norm):
    g = torch.Generator().manual_seed(11)
    n, e, k, scale = 6, 10, 3, 2.5
    logits = torch.randn(n, e, generator=g, dtype=torch.float64)
    w = torch.randn(n, k, generator=g, dtype=torch.float64)
    cfg = R.RouterCfg(num_experts=e, top_k=k, score_func=sf, route_norm=norm, route_scale=scale)
    _, idx, _, _ = R.router_forward(logits.float(), None, cfg)

    def f(lg):
        s = R.score_fn(lg, sf).gather(1, idx)
        if norm:
            s = s / (s.sum(-1, keepdim=True) + 1e-20)
        return (s * scale * w).sum()

    lg = logits.clone().requires_grad_(True)
    f(lg).backward()
    eps = 1e-6
    fd = torch.zeros_like(logits)
    for i in range(n):
        for j in range(e):
            p, m = logits.clone(), logits.clone()
            p[i, j] += eps
            m[i, j] -= eps
            fd[i, j] = (f(p) - f(m)) / (2 * eps)
    torch.testing.assert_close(lg.grad, fd, rtol=1e-6, atol=1e-8)


# ---------------------------------------------------------------------------
# whole layer vs the reference op sequence
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("score_before,grouped", [(True, False), (False, False), (True, True)])
def test_moe_forward_matches_reference_op_sequence(score_before, grouped):
    g = torch.Generator().manual_seed(12)
    bs, slen, d, e, k, h, hs = 2, 24, 32, 8, 2, 48, 40
    params = {
        "gate": torch.randn(e, d, generator=g) * 0.1,
        "w1": torch.randn(e, h, d, generator=g) * 0.05, "w2": torch.randn(e, d, h, generator=g) * 0.05,
        "w3": torch.randn(e, h, d, generator=g) * 0.05,
        "sw1": torch.randn(hs, d, generator=g) * 0.05, "sw2": torch.randn(d, hs, generator=g) * 0.05,
        "sw3": torch.randn(hs, d, generator=g) * 0.05, "expert_bias": torch.rand(e, generator=g) * 0.02 - 0.01,
    }
    x = torch.randn(bs, slen, d, generator=g)
    gout = torch.randn(bs, slen, d, generator=g)
    rc = R.RouterCfg(num_experts=e, top_k=k, score_func="softmax", route_norm=True, route_scale=1.5)
    cfg = R.MoECfg(router=rc, dim=d, hidden_dim=h, score_before_experts=score_before,
                   use_grouped_mm=grouped, has_shared=True)
    outs, grads = [], []
    for fn in (R.moe_forward, R.moe_forward_reference_ops):
        p = {n: t.clone().requires_grad_(n != "expert_bias") for n, t in params.items()}
        xi = x.clone().requires_grad_(True)
        out = fn(p, xi, cfg)
        out.backward(gout)
        outs.append(out.detach())
        grads.append([xi.grad] + [p[n].grad for n in ("gate", "w1", "w2", "w3", "sw1")])
    tol = dict(rtol=2e-2, atol=2e-2) if grouped else dict(rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(outs[0], outs[1], **tol)
    for a, b in zip(grads[0], grads[1]):
        torch.testing.assert_close(a, b, **tol)


def test_reference_ops_logit_values_override():
    """logit_values replaces the gate logits' values only: the same values give the
    same output and gradients; values an ulp away keep the gate in the gradient
    path; values further off than fp32 summation order are refused."""
    g = torch.Generator().manual_seed(5)
    bs, slen, d, e, k, h = 2, 16, 32, 8, 2, 48
    params = {"gate": torch.randn(e, d, generator=g) * 0.1, "w1": torch.randn(e, h, d, generator=g) * 0.05,
              "w2": torch.randn(e, d, h, generator=g) * 0.05, "w3": torch.randn(e, h, d, generator=g) * 0.05}
    x = torch.randn(bs, slen, d, generator=g)
    gout = torch.randn(bs, slen, d, generator=g)
    rc = R.RouterCfg(num_experts=e, top_k=k, score_func="sigmoid", route_norm=True, route_scale=1.0)
    cfg = R.MoECfg(router=rc, dim=d, hidden_dim=h, score_before_experts=False, use_grouped_mm=False,
                   has_shared=False)
    logits = x.view(-1, d) @ params["gate"].t()

    def run(values):
        p = {n: t.clone().requires_grad_(True) for n, t in params.items()}
        xi = x.clone().requires_grad_(True)
        out = R.moe_forward_reference_ops(p, xi, cfg, logit_values=values)
        out.backward(gout)
        return out.detach(), xi.grad, p["gate"].grad

    base = run(None)
    same = run(logits.clone())
    for a, b in zip(base, same):
        assert torch.equal(a, b)
    nudged = logits.clone()
    nudged[0, 0] = torch.nextafter(nudged[0, 0], torch.tensor(float("inf")))
    out_n, dx_n, dgate_n = run(nudged)
    assert dgate_n is not None and torch.count_nonzero(dgate_n) > 0
    torch.testing.assert_close(dgate_n, base[2], rtol=1e-4, atol=1e-6)
    with pytest.raises(AssertionError, match="differ from the fp32 gate GEMM"):
        run(logits + 1e-3 * logits.abs().max())


# ---------------------------------------------------------------------------
# aux-loss-free bias update: hand-worked closed forms (optimizer.py:416-431)
# ---------------------------------------------------------------------------


def _bias_case(t, coeff=1e-3, halve=False, bias=None):
    tt = torch.tensor(t, dtype=torch.float32)
    b = torch.zeros(len(t)) if bias is None else torch.tensor(bias, dtype=torch.float32)
    R.expert_bias_update([tt], [b], [coeff], [halve])
    assert torch.count_nonzero(tt) == 0
    return b


def test_bias_update_balanced_is_noop():
    assert torch.equal(_bias_case([7.0, 7.0, 7.0, 7.0], bias=[0.5, -0.5, 0.25, 0.0]),
                       torch.tensor([0.5, -0.5, 0.25, 0.0]))


def test_bias_update_one_hot_expert():
    # mean 4: signs (-1, 1, 1, 1); mean of delta = coeff / 2
    c = torch.tensor(0.125)  # a power of two keeps every step exact
    b = _bias_case([10.0, 2.0, 2.0, 2.0], coeff=float(c))
    assert torch.equal(b, torch.tensor([-1.5, 0.5, 0.5, 0.5]) * c)


def test_bias_update_ties_with_mean_get_zero_sign():
    # mean 3: signs (1, 0, -1, 0) -> mean 0
    b = _bias_case([2.0, 3.0, 4.0, 3.0], coeff=0.25)
    assert torch.equal(b, torch.tensor([0.25, 0.0, -0.25, 0.0]))


def test_bias_update_recompute_halves_with_floor():
    # [9, 3, 3, 1] // 2 = [4, 1, 1, 0], mean 1.5: signs (-1, 1, 1, 1)
    b = _bias_case([9.0, 3.0, 3.0, 1.0], coeff=0.5, halve=True)
    assert torch.equal(b, torch.tensor([-0.75, 0.25, 0.25, 0.25]))


@pytest.mark.parametrize("pad", [1, 16, 32])
def test_permute_pad_layout_reduces_to_the_unpadded_permute(pad):
    """The padded layout (fixed by TorchAOExpertParallel's call site) holds the
    unpadded permutation's rows in order, each expert group padded to a multiple of
    pad with the appended zero row's index, and is the unpadded one for pad = 1."""
    rng = np.random.default_rng(pad)
    for ranks, experts in [(1, 4), (3, 5), (8, 2)]:
        counts = rng.integers(0, 40, ranks * experts)
        idx, ntok = R.generate_permute_indices(counts, experts, ranks)
        pidx, padded, ends = R.generate_permute_pad_indices(counts, experts, ranks, pad)
        n_in = int(counts.sum())
        assert np.array_equal(pidx[pidx != n_in], idx)
        assert all(p % pad == 0 and p >= g for p, g in zip(padded, ntok))
        assert np.array_equal(ends, np.cumsum(padded)) and len(pidx) == ends[-1]
        starts = np.concatenate([[0], ends[:-1]])
        for e in range(experts):
            grp = pidx[starts[e]:ends[e]]
            assert np.all(grp[ntok[e]:] == n_in) and np.all(grp[:ntok[e]] != n_in)
        if pad == 1:
            assert np.array_equal(pidx, idx)


# ---------------------------------------------------------------------------
# MXFP8 quantization (torchao's to_mx, RCEIL) and the MX GEMM emulation
# ---------------------------------------------------------------------------


def _rceil_bits(amax: float) -> int:
    """RCEIL e8m0 exponent from the fp32 bits of amax / 448: the biased exponent,
    plus one when the mantissa is non-zero; subnormals above 2^-127 give 1."""
    d = np.float32(amax) / np.float32(448.0)
    if np.isnan(d):
        return 255
    b = int(np.array([d], dtype=np.float32).view(np.uint32)[0])
    if b >= 0x7F800000:
        return 254
    ex, man = b >> 23, b & 0x7FFFFF
    if ex == 0:
        return 1 if man > 0x400000 else 0
    return min(ex + (man != 0), 254)


def _e4m3_grid() -> torch.Tensor:
    """Every finite non-negative float8_e4m3fn value (bytes 0x00..0x7e)."""
    return torch.arange(0, 0x7F, dtype=torch.uint8).view(torch.float8_e4m3fn).float()


def test_mx_exponent_matches_bit_derivation():
    g = torch.Generator().manual_seed(0)
    vals = [0.0, 448.0, 449.0, 450.0, 447.0, 1.0, 3.5, 224.0, 896.0]
    vals += [448.0 * 2.0 ** k for k in range(-125, 120, 7)]
    vals += (torch.randn(400, generator=g).abs() * torch.exp2(torch.randint(-120, 110, (400,), generator=g).float())
             ).bfloat16().float().tolist()
    vals += [2.0 ** -120, 2.0 ** -126 * 448.0 * 1.5, 2.0 ** -127 * 448.0]
    x = torch.zeros(len(vals), 32)
    x[:, 5] = torch.tensor(vals)
    _, e = R.quant_mxfp8(x.bfloat16())
    bf = x.bfloat16().float()[:, 5]
    want = torch.tensor([_rceil_bits(v) for v in bf.tolist()], dtype=torch.uint8)
    assert torch.equal(e.view(-1), want)


def test_mx_hand_worked_blocks():
    x = torch.zeros(4, 64)
    x[0, 0], x[0, 1], x[0, 2] = 448.0, 1.0, -3.0   # amax 448: e = 127, values kept
    x[1, 0], x[1, 1] = 450.0, 3.0                  # 450 / 448 > 1: e = 128, values halved
    x[1, 40] = 0.5                                 # second block: 0.5 / 448 = 2^-9.8 -> ceil -9 -> e = 118
    x[2, 33] = 2.0 ** -120                         # ceil(log2) < -127: e = 0 and multiplier 1 -> q = 0
    q, e = R.quant_mxfp8(x.bfloat16())
    qf = q.float()
    assert e.tolist() == [[127, 0], [128, 118], [0, 0], [0, 0]]
    assert qf[0, :3].tolist() == [448.0, 1.0, -3.0]
    assert qf[1, :2].tolist() == [224.0, 1.5]      # 225 rounds to the e4m3 step 224
    assert qf[1, 40].item() == 256.0               # 0.5 * 2^9
    assert torch.count_nonzero(qf[2]) == 0 and torch.count_nonzero(qf[3]) == 0
    nan = torch.zeros(1, 32)
    nan[0, 3] = float("nan")
    assert R.quant_mxfp8(nan.bfloat16())[1].item() == 255


def test_mx_grid_round_trip_and_equivariance():
    grid = _e4m3_grid()
    g = torch.Generator().manual_seed(1)
    blocks = grid[torch.randint(0, len(grid), (64, 32), generator=g)] * torch.where(
        torch.rand(64, 32, generator=g) < 0.5, -1.0, 1.0)
    blocks[:, 7] = 448.0  # amax 448: e = 127, grid values are exact
    q, e = R.quant_mxfp8(blocks.bfloat16())
    assert torch.equal(e, torch.full((64, 1), 127, dtype=torch.uint8))
    assert torch.equal(q.float(), blocks)
    for k in (-100, -7, 1, 60):
        qk, ek = R.quant_mxfp8((blocks * 2.0 ** k).bfloat16())
        assert torch.equal(qk.float(), blocks) and torch.equal(ek.long(), e.long() + k)


def test_mx_rounding_bound_and_block_locality():
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(50, 256, generator=g) * torch.exp(torch.randn(50, 8, generator=g) * 4).repeat_interleave(32, 1)
         ).bfloat16()
    q, e = R.quant_mxfp8(x)
    deq = R.mx_dequant(q, e)
    xf = x.double()
    step = torch.ldexp(torch.ones(e.shape, dtype=torch.float64), e.double() - 127 - 10).repeat_interleave(32, 1)
    assert ((deq - xf).abs() <= torch.maximum(xf.abs() * 2.0 ** -4, step)).all()
    # blocks along the other dimension: the transposed quantization
    qt, et = R.quant_mxfp8(x.t().contiguous(), dim=0)
    assert torch.equal(qt.float(), q.float().t()) and torch.equal(et, e.t())
    # changing one element moves only its own block's scale
    y = x.clone()
    y[3, 70] = 1e4
    _, e2 = R.quant_mxfp8(y)
    diff = (e2 != e).nonzero().tolist()
    assert diff == [[3, 2]]


def test_mx_mm_exact_on_grid_values_with_block_scales():
    grid = _e4m3_grid()
    g = torch.Generator().manual_seed(3)
    a = grid[torch.randint(0, len(grid), (5, 96), generator=g)]
    b = grid[torch.randint(0, len(grid), (7, 96), generator=g)] * -1.0
    a[:, 0::32] = 448.0
    b[:, 0::32] = -448.0
    ka = torch.tensor([-3.0, 0.0, 5.0]).repeat_interleave(32)  # different power-of-two per block
    kb = torch.tensor([2.0, -6.0, 1.0]).repeat_interleave(32)
    xa, xb = a * torch.exp2(ka), b * torch.exp2(kb)
    qa, sa = R.quant_mxfp8(xa.bfloat16())
    qb, sb = R.quant_mxfp8(xb.bfloat16())
    assert sa[0].tolist() == [124, 127, 132] and sb[0].tolist() == [129, 121, 128]
    assert torch.equal(R.mx_dequant(qa, sa), xa.double()) and torch.equal(R.mx_dequant(qb, sb), xb.double())
    assert torch.equal(R._mx_mm(qa, sa, qb, sb), (xa.double() @ xb.double().t()).float())


def test_mx_experts_close_to_bf16_reference():
    g = torch.Generator().manual_seed(4)
    e, d, h, counts = 3, 64, 96, [20, 0, 45]
    r = sum(counts)
    x = torch.randn(r, d, generator=g).bfloat16()
    w1, w3 = ((torch.randn(e, h, d, generator=g) * 0.1).bfloat16() for _ in range(2))
    w2 = (torch.randn(e, d, h, generator=g) * 0.1).bfloat16()
    dy = torch.randn(r, d, generator=g).bfloat16()
    cnt = torch.tensor(counts)
    y, g_, u_, h_ = R.experts_mxfp8_forward(w1, w2, w3, x, cnt)
    dx, dw1, dw2, dw3 = R.experts_mxfp8_backward(w1, w2, w3, x, cnt, g_, u_, h_, dy)
    xr, w1r, w2r, w3r = (t.double().requires_grad_(True) for t in (x, w1, w2, w3))
    ys, s0 = [], 0
    for i, c in enumerate(counts):
        xe = xr[s0:s0 + c]
        ys.append((F.silu(xe @ w1r[i].t()) * (xe @ w3r[i].t())) @ w2r[i].t())
        s0 += c
    yr = torch.cat(ys)
    yr.backward(dy.double())

    def rel(a, b):
        return ((a.double() - b).abs().max() / b.abs().max()).item()
    errs = [rel(y, yr.detach()), rel(dx, xr.grad), rel(dw1, w1r.grad), rel(dw2, w2r.grad), rel(dw3, w3r.grad)]
    assert max(errs) < 0.1, errs
    assert torch.count_nonzero(dw1[1]) == 0 and torch.count_nonzero(dw2[1]) == 0


# ---------------------------------------------------------------------------
# gpt-oss experts (gpt_oss/moe.py:43-122)
# ---------------------------------------------------------------------------


def test_oss_swiglu_hand_worked_values():
    import math

    L, a = 7.0, 1.702
    h1 = torch.tensor([[10.0, -9.0, -3.0, 0.5, 2.0, 8.0, 7.0, -7.0]], dtype=torch.float64)
    out = R.oss_swiglu(h1, L)[0].tolist()

    def sig(z):
        return 1.0 / (1.0 + math.exp(-z))
    want = [7.0 * sig(a * 7.0) * (-7.0 + 1.0),   # glu clamped to 7, linear clamped to -7
            -3.0 * sig(-3.0 * a) * 1.5,          # no clamp; the glu is not clamped from below
            2.0 * sig(2.0 * a) * (7.0 + 1.0),    # linear clamped to +7
            7.0 * sig(7.0 * a) * (-7.0 + 1.0)]   # exactly at the limits
    assert out == pytest.approx(want, rel=1e-12)


def test_oss_swiglu_gradient_masks_and_finite_differences():
    L = 7.0
    h1 = torch.tensor([[10.0, -9.0, -3.0, 0.5, 6.5, 7.5, -2.0, -6.0]], dtype=torch.float64, requires_grad=True)
    R.oss_swiglu(h1, L).sum().backward()
    gr = h1.grad[0]
    assert gr[0] == 0 and gr[1] == 0 and gr[5] == 0      # clamped inputs get no gradient
    assert gr[2] != 0 and gr[3] != 0 and gr[4] != 0 and gr[6] != 0 and gr[7] != 0
    eps = 1e-6
    for i in (2, 3, 4, 6, 7):
        hp, hm = h1.detach().clone(), h1.detach().clone()
        hp[0, i] += eps
        hm[0, i] -= eps
        fd = (R.oss_swiglu(hp, L).sum() - R.oss_swiglu(hm, L).sum()) / (2 * eps)
        assert gr[i].item() == pytest.approx(fd.item(), rel=1e-6)


def test_oss_grouped_mm_matches_for_loop_and_float64():
    g = torch.Generator().manual_seed(5)
    e, d, h = 4, 64, 48
    cnt = torch.tensor([9, 0, 17, 4])
    r = int(cnt.sum())
    x = torch.randn(r, d, generator=g).bfloat16()
    w1 = (torch.randn(e, 2 * h, d, generator=g) * 0.3).bfloat16()
    b1 = torch.randn(e, 2 * h, generator=g).bfloat16()
    w2 = (torch.randn(e, d, h, generator=g) * 0.3).bfloat16()
    b2 = torch.randn(e, d, generator=g).bfloat16()
    grouped = R.oss_experts_grouped_mm(w1, b1, w2, b2, 7.0, x, cnt)
    loop = R.oss_experts_for_loop(w1, b1, w2, b2, 7.0, x, cnt)
    assert torch.equal(grouped, loop)
    f64 = R.oss_experts_for_loop(w1.double(), b1.double(), w2.double(), b2.double(), 7.0, x.double(), cnt)
    assert ((grouped.double() - f64).abs().max() / f64.abs().max()).item() < 2e-2


# ---------------------------------------------------------------------------
# fp8 rowwise quantization: power-of-two scales and the e4m3 rounding
# ---------------------------------------------------------------------------


def test_fp8_scale_known_answers():
    """s = 2^-floor(log2(448 / max(amax, 1e-12))), worked by hand."""
    amax = torch.tensor([1.0, 448.0, 0.5, 0.0, 3.0, 7.0 * 2.0 ** -10, 1e30, 449.0, 224.0, 223.0])
    want = torch.tensor([2.0 ** -8,   # 448 / 1 = 448 in [256, 512)
                         1.0,         # exactly 1
                         2.0 ** -9,   # 896 in [512, 1024)
                         2.0 ** -48,  # 448e12 in [2^48, 2^49)
                         2.0 ** -7,   # 149.3 in [128, 256)
                         2.0 ** -16,  # exactly 2^16
                         2.0 ** 91,   # 4.48e-28 in [2^-91, 2^-90)
                         2.0,         # 0.998 in [0.5, 1)
                         0.5,         # exactly 2
                         0.5])        # 2.009 in [2, 4)
    got = R.fp8_scale(amax)
    assert torch.equal(got, want), (got, want)


def test_fp8_scale_range_and_power_of_two():
    """Over 30 decades of amax above the 1e-12 floor: s is a power of two and
    amax / s lies in (224, 448]."""
    g = torch.Generator().manual_seed(9)
    amax = torch.exp(torch.empty(20000).uniform_(-27.0, 46.0, generator=g)).bfloat16().float()
    s = R.fp8_scale(amax)
    mant, _ = torch.frexp(s)
    assert torch.all(mant == 0.5)
    r = amax / s
    assert torch.all(r <= 448.0) and torch.all(r > 224.0)


def _e4m3fn_rne_codes(v: np.ndarray) -> np.ndarray:
    """Independent OCP e4m3fn encoder for |v| <= 448: the nearest of the 127 finite
    non-negative codes (bias 7, 3 mantissa bits, subnormals 2^-9 apart), ties to
    the even code, sign in bit 7."""
    codes = np.arange(0x7F)
    ex, m = codes >> 3, codes & 7
    vals = np.where(ex == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (ex - 7.0))
    a = np.abs(v.astype(np.float64))[:, None]
    d = np.abs(vals[None, :] - a)
    best = d.min(axis=1, keepdims=True)
    cand = np.where(d == best, codes[None, :], 1 << 10)
    even = np.where((cand & 1) == 0, cand, 1 << 10).min(axis=1)
    pick = np.where(even < (1 << 10), even, cand.min(axis=1))
    return (pick | np.where(np.signbit(v), 0x80, 0)).astype(np.uint8)


def test_fp8_cast_matches_independent_e4m3_encoder():
    """torch's float8_e4m3fn cast, which quant_fp8_rows applies to x / s, equals an
    independent round-to-nearest-even encoder on every bf16 value in [-448, 448]."""
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    v = bits.float()
    v = v[torch.isfinite(v) & (v.abs() <= 448.0)]
    got = v.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    want = _e4m3fn_rne_codes(v.numpy())
    # -0.0 encodes as 0x80 in both
    assert np.array_equal(got, want)


def test_quant_fp8_rows_rounding_bound():
    """Each dequantized value q * s is x rounded to the e4m3 grid scaled by s:
    within half an e4m3 spacing of x / s, and the row's amax lands in (224, 448]."""
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(64, 96, generator=g) * torch.exp(torch.empty(64, 1).uniform_(-20, 20, generator=g))).bfloat16()
    q, s = R.quant_fp8_rows(x)
    y = x.float() / s
    back = q.float()
    a = y.abs().clamp_min(2.0 ** -6)
    half_spacing = torch.exp2(torch.floor(torch.log2(a)) - 4)
    assert torch.all((back - y).abs() <= half_spacing)
    assert torch.all(y.abs().amax(dim=1) > 224.0) and torch.all(y.abs().amax(dim=1) <= 448.0)


# ---------------------------------------------------------------------------
# fp8 expert emulation (experts_fp8_forward / experts_fp8_backward): each GEMM is
# pinned by operands on the e4m3 grid carrying power-of-two scales along the
# axis the recipe scales (per token row, per expert output column, per column
# over a group's tokens for dW): quantization is then exact and every GEMM must
# equal the fp64 product rounded once. A scale taken along the contraction
# breaks that, which the planted-mistake tests check.
# ---------------------------------------------------------------------------


def _grid_rows(rows: int, cols: int, g: torch.Generator, kmin: int = -5, kmax: int = 5) -> torch.Tensor:
    """[rows, cols] bf16: e4m3 grid values with random signs, one +-448 per row,
    each row times its own power of two 2^k, k in [kmin, kmax]."""
    grid = _e4m3_grid()
    v = grid[torch.randint(0, len(grid), (rows, cols), generator=g)]
    v = v * torch.where(torch.rand(rows, cols, generator=g) < 0.5, -1.0, 1.0)
    v[torch.arange(rows), torch.randint(0, cols, (rows,), generator=g)] = 448.0
    k = torch.randint(kmin, kmax + 1, (rows, 1), generator=g).float()
    return (v * torch.exp2(k)).bfloat16()


def _both_ways_exact(rows: int, cols: int, g: torch.Generator) -> torch.Tensor:
    """[rows, cols] bf16 grid values with a 448 in every row and every column, so
    that quantizing along either axis has scale 1 and is exact."""
    v = _grid_rows(rows, cols, g, 0, 0).float()
    v[torch.randint(0, rows, (cols,), generator=g), torch.arange(cols)] = -448.0
    return v.bfloat16()


def _bf16_mm64(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a @ b in fp64, rounded to fp32 and then bf16 (the emulation's rounding)."""
    return (a.double() @ b.double()).float().bfloat16()


def _deq(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    return q.double() * s.double()


def _fp8_forward_mismatches(e, d, h, counts, seed) -> int:
    """Runs experts_fp8_forward on grid operands (x scaled per token row, w1 / w3
    per (expert, hidden row) over D, w2 per (expert, dim row) over H) and counts
    elements of g, u, y that differ from the fp64 products: g, u of the inputs
    themselves, y of h dequantized by the pinned row quantizer."""
    g = torch.Generator().manual_seed(seed)
    r = sum(counts)
    x = _grid_rows(r, d, g)
    w1 = torch.stack([_grid_rows(h, d, g) for _ in range(e)])
    w3 = torch.stack([_grid_rows(h, d, g) for _ in range(e)])
    w2 = torch.stack([_grid_rows(d, h, g) for _ in range(e)])
    y, gg, uu, hh = R.experts_fp8_forward(w1, w2, w3, x, torch.tensor(counts))
    qh, sh = R.quant_fp8_rows(hh)
    hd = _deq(qh, sh)
    bad, s0 = 0, 0
    for i, c in enumerate(counts):
        sl = slice(s0, s0 + c)
        bad += int((gg[sl] != _bf16_mm64(x[sl], w1[i].t())).sum())
        bad += int((uu[sl] != _bf16_mm64(x[sl], w3[i].t())).sum())
        bad += int((y[sl] != _bf16_mm64(hd[sl], w2[i].t())).sum())
        s0 += c
    assert torch.equal(hh, F.silu(gg) * uu)
    return bad


def _fp8_backward_mismatches(e, d, h, counts, seed) -> dict:
    """Runs experts_fp8_backward twice on grid operands and counts mismatches
    against fp64 products, with the SwiGLU gradient from torch's autograd:
      dx: dy per token row, w2 per (expert, hidden row) over D, w1 / w3 per
          (expert, dim column) over H; dg, du dequantized per token row;
      dW: dy exact both ways (scale 1), x and h per column over each expert's
          tokens; dg, du dequantized per column over the tokens."""
    g = torch.Generator().manual_seed(seed)
    r = sum(counts)
    cnt = torch.tensor(counts)
    bad = {"dx": 0, "dw1": 0, "dw2": 0, "dw3": 0}

    def swiglu_grads(gs, us, dh):
        gq, uq = gs.clone().requires_grad_(True), us.clone().requires_grad_(True)
        (F.silu(gq) * uq).backward(dh)
        return gq.grad, uq.grad

    # --- dx ---
    dy = _grid_rows(r, d, g)
    w2 = torch.stack([_grid_rows(h, d, g).t() for _ in range(e)])  # [E, D, H], rows of w2^T on the grid
    w1 = torch.stack([_grid_rows(d, h, g).t() for _ in range(e)])  # [E, H, D], rows of w1^T on the grid
    w3 = torch.stack([_grid_rows(d, h, g).t() for _ in range(e)])
    gs = torch.randn(r, h, generator=g).bfloat16()
    us = torch.randn(r, h, generator=g).bfloat16()
    hs = F.silu(gs) * us
    x = torch.randn(r, d, generator=g).bfloat16()
    dx, *_ = R.experts_fp8_backward(w1, w2, w3, x, cnt, gs, us, hs, dy)
    s0 = 0
    dgs, dus = [], []
    for i, c in enumerate(counts):
        sl = slice(s0, s0 + c)
        dg, du = swiglu_grads(gs[sl], us[sl], _bf16_mm64(dy[sl], w2[i]))
        dgs.append(dg)
        dus.append(du)
        s0 += c
    dg, du = torch.cat(dgs), torch.cat(dus)
    dgd, dud = _deq(*R.quant_fp8_rows(dg)), _deq(*R.quant_fp8_rows(du))
    s0 = 0
    for i, c in enumerate(counts):
        sl = slice(s0, s0 + c)
        want = _bf16_mm64(dgd[sl], w1[i]) + _bf16_mm64(dud[sl], w3[i])
        bad["dx"] += int((dx[sl] != want).sum())
        s0 += c

    # --- dW ---
    segs = [c for c in counts if c]
    dy = torch.cat([_both_ways_exact(c, d, g) for c in segs]) if segs else torch.zeros(0, d).bfloat16()
    x = torch.cat([_grid_rows(d, c, g).t() for c in segs]) if segs else torch.zeros(0, d).bfloat16()
    hs = torch.cat([_grid_rows(h, c, g).t() for c in segs]) if segs else torch.zeros(0, h).bfloat16()
    gs = torch.randn(r, h, generator=g).bfloat16()
    us = torch.randn(r, h, generator=g).bfloat16()
    w2 = torch.stack([_grid_rows(h, d, g).t() for _ in range(e)])
    w1 = torch.randn(e, h, d, generator=g).bfloat16()
    w3 = torch.randn(e, h, d, generator=g).bfloat16()
    _, dw1, dw2, dw3 = R.experts_fp8_backward(w1, w2, w3, x, cnt, gs, us, hs, dy)
    s0 = 0
    for i, c in enumerate(counts):
        sl = slice(s0, s0 + c)
        if c == 0:
            for name, t in (("dw1", dw1), ("dw2", dw2), ("dw3", dw3)):
                bad[name] += int(torch.count_nonzero(t[i]))
            continue
        dg, du = swiglu_grads(gs[sl], us[sl], _bf16_mm64(dy[sl], w2[i]))
        dgc = _deq(*R.quant_fp8_rows(dg.t()))  # [H, c]: one scale per hidden column over the tokens
        duc = _deq(*R.quant_fp8_rows(du.t()))
        bad["dw1"] += int((dw1[i] != _bf16_mm64(dgc, x[sl])).sum())
        bad["dw3"] += int((dw3[i] != _bf16_mm64(duc, x[sl])).sum())
        bad["dw2"] += int((dw2[i] != _bf16_mm64(dy[sl].t(), hs[sl])).sum())
        s0 += c
    return bad


def test_fp8_forward_exact_on_grid_operands():
    assert _fp8_forward_mismatches(3, 64, 96, [20, 0, 45], seed=11) == 0


def test_fp8_backward_exact_on_grid_operands():
    bad = _fp8_backward_mismatches(3, 64, 96, [20, 0, 45], seed=12)
    assert bad == {"dx": 0, "dw1": 0, "dw2": 0, "dw3": 0}, bad


def test_fp8_pins_catch_weights_scaled_along_the_contraction(monkeypatch):
    """Planted mistake: the expert weights scaled per (expert, contraction index)
    instead of per output column. Square shapes let the wrong scales broadcast
    silently; the grid pin must see the difference."""
    assert _fp8_forward_mismatches(2, 64, 64, [64, 64], seed=13) == 0
    orig = R.quant_fp8_rows
    monkeypatch.setattr(R, "quant_fp8_rows", lambda t, dim=-1: orig(t, dim=-2 if t.dim() == 3 else dim))
    assert _fp8_forward_mismatches(2, 64, 64, [64, 64], seed=13) > 0


def test_fp8_pins_catch_transposed_operand_scales(monkeypatch):
    """Planted mistake: every transposed operand of the backward (w1^T, w2^T, w3^T
    and the dW operands) scaled along the other axis, i.e. along the
    contraction. Both the dx and the dW pins must see it."""
    assert _fp8_backward_mismatches(2, 64, 64, [64, 64], seed=14) == {"dx": 0, "dw1": 0, "dw2": 0, "dw3": 0}
    orig = R.quant_fp8_rows
    monkeypatch.setattr(R, "quant_fp8_rows",
                        lambda t, dim=-1: orig(t, dim=0 if (t.dim() == 2 and not t.is_contiguous()) else dim))
    bad = _fp8_backward_mismatches(2, 64, 64, [64, 64], seed=14)
    assert bad["dx"] > 0 and bad["dw1"] > 0 and bad["dw2"] > 0 and bad["dw3"] > 0, bad


def test_fp8_experts_close_to_float64_reference():
    """Forward and backward of the fp8 emulation within 0.1 (normwise relative,
    max |ours - ref| / max |ref|) of an fp64 autograd reference of the same
    bf16 operands; empty experts get zero weight gradients."""
    g = torch.Generator().manual_seed(15)
    e, d, h, counts = 3, 64, 96, [20, 0, 45]
    r = sum(counts)
    x = torch.randn(r, d, generator=g).bfloat16()
    w1, w3 = ((torch.randn(e, h, d, generator=g) * 0.1).bfloat16() for _ in range(2))
    w2 = (torch.randn(e, d, h, generator=g) * 0.1).bfloat16()
    dy = torch.randn(r, d, generator=g).bfloat16()
    cnt = torch.tensor(counts)
    y, g_, u_, h_ = R.experts_fp8_forward(w1, w2, w3, x, cnt)
    dx, dw1, dw2, dw3 = R.experts_fp8_backward(w1, w2, w3, x, cnt, g_, u_, h_, dy)
    xr, w1r, w2r, w3r = (t.double().requires_grad_(True) for t in (x, w1, w2, w3))
    ys, s0 = [], 0
    for i, c in enumerate(counts):
        xe = xr[s0:s0 + c]
        ys.append((F.silu(xe @ w1r[i].t()) * (xe @ w3r[i].t())) @ w2r[i].t())
        s0 += c
    yr = torch.cat(ys)
    yr.backward(dy.double())

    def rel(a, b):
        return ((a.double() - b).abs().max() / b.abs().max()).item()
    errs = [rel(y, yr.detach()), rel(dx, xr.grad), rel(dw1, w1r.grad), rel(dw2, w2r.grad), rel(dw3, w3r.grad)]
    assert max(errs) < 0.1, errs
    assert torch.count_nonzero(dw1[1]) == 0 and torch.count_nonzero(dw2[1]) == 0
