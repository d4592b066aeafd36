"""The MoE layer's glue (torchtitan/models/common/moe.py:380-477) pinned
independently of the oracle's restatements, on the CPU in fp64.

Every piece of the layer (router, reorder, experts, combine) is pinned by its
own tests; this pins how MoE.forward composes them. The gate weights are built
so that the routing is known by construction (the gate reads one coordinate per
expert, whose planted values order the experts, and one expert's bias is large
enough that the choice always takes it while its score stays the unbiased
sigmoid), and the layer's output is written directly from the definition:

    out[t] = shared(x_t) + sum over chosen e of  FFN_e(s_te x_t)   (score before the experts)
                                            or  s_te FFN_e(x_t)    (score after them)
    s_te = route_scale * sigmoid(l_te) / (sum over chosen e' of sigmoid(l_te') + 1e-20)

with FFN_e(v) = w2_e (silu(w1_e v) * (w3_e v)). Both restatements
(moe_forward_reference_ops, the reference's op sequence, and moe_forward) must
equal it; versions of the op sequence with a planted mistake (the score on the
other side of the experts, token = perm % K, the shared output dropped, the
score gathered from the biased choice) must not.
"""

import inspect
import textwrap

import pytest
import torch
import torch.nn.functional as F

from oracle import moe_ref as R

E, D, H, HS, N = 4, 8, 6, 5, 12
ROUTE_SCALE = 2.5
GATE_GAIN = 3.0
LEVELS = torch.tensor([-1.0, -0.3, 0.4, 1.1], dtype=torch.float64)
BIASED_EXPERT, BIAS = 1, 5.0


def _case(seed: int, shared: bool):
    g = torch.Generator().manual_seed(seed)
    perms = torch.stack([torch.randperm(E, generator=g) for _ in range(N)])
    x = torch.randn(N, D, generator=g, dtype=torch.float64)
    x[:, :E] = LEVELS[perms]  # token t offers expert e the level of rank perms[t, e]
    gate = torch.zeros(E, D, dtype=torch.float64)
    gate[range(E), range(E)] = GATE_GAIN
    bias = torch.zeros(E, dtype=torch.float32)
    bias[BIASED_EXPERT] = BIAS
    p = {
        "gate": gate,
        "expert_bias": bias,
        "w1": torch.randn(E, H, D, generator=g, dtype=torch.float64) * 0.7,
        "w2": torch.randn(E, D, H, generator=g, dtype=torch.float64) * 0.7,
        "w3": torch.randn(E, H, D, generator=g, dtype=torch.float64) * 0.7,
    }
    if shared:
        p.update(sw1=torch.randn(HS, D, generator=g, dtype=torch.float64) * 0.7,
                 sw2=torch.randn(D, HS, generator=g, dtype=torch.float64) * 0.7,
                 sw3=torch.randn(HS, D, generator=g, dtype=torch.float64) * 0.7)
    return x, p


def _chosen(x_t: torch.Tensor, k: int) -> list[int]:
    """The experts token t routes to, from the construction alone: the biased
    expert (its bias exceeds every score gap), then the highest planted levels."""
    rest = sorted((e for e in range(E) if e != BIASED_EXPERT), key=lambda e: -float(x_t[e]))
    return [BIASED_EXPERT] + rest[: k - 1]


def _ffn(w1, w2, w3, v):
    return w2 @ (F.silu(w1 @ v) * (w3 @ v))


def _direct(x: torch.Tensor, p: dict, k: int, score_before: bool, shared: bool) -> torch.Tensor:
    out = torch.zeros_like(x)
    for t in range(N):
        xt = x[t]
        if shared:
            out[t] += _ffn(p["sw1"], p["sw2"], p["sw3"], xt)
        chosen = _chosen(xt, k)
        sig = {e: torch.sigmoid(GATE_GAIN * xt[e]) for e in chosen}
        den = sum(sig.values()) + 1e-20
        for e in chosen:
            s = ROUTE_SCALE * sig[e] / den
            w = (p["w1"][e], p["w2"][e], p["w3"][e])
            out[t] += _ffn(*w, s * xt) if score_before else s * _ffn(*w, xt)
    return out


def _cfg(k: int, score_before: bool, shared: bool) -> R.MoECfg:
    rc = R.RouterCfg(num_experts=E, top_k=k, score_func="sigmoid", route_norm=True, route_scale=ROUTE_SCALE)
    return R.MoECfg(router=rc, dim=D, hidden_dim=H, score_before_experts=score_before, use_grouped_mm=False,
                    has_shared=shared)


CASES = [(k, sb, sh) for k in (1, 2, 3) for sb in (True, False) for sh in (True, False)]


def _close(a: torch.Tensor, b: torch.Tensor) -> bool:
    # the restatements round routed rows and the combine's sums through fp32
    return bool((a - b).abs().max() <= 1e-5 * b.abs().max())


@pytest.mark.parametrize("k,score_before,shared", CASES)
def test_layer_equals_its_definition(k, score_before, shared):
    x, p = _case(seed=10 * k + 2 * score_before + shared, shared=shared)
    want = _direct(x, p, k, score_before, shared)
    cfg = _cfg(k, score_before, shared)
    aux = {}
    got_ops = R.moe_forward_reference_ops(p, x.view(1, N, D), cfg).view(N, D)
    got = R.moe_forward(p, x.view(1, N, D), cfg, aux=aux).view(N, D)
    # the construction's routing is the one the restatement took
    for t in range(N):
        assert sorted(aux["idx"][t].tolist()) == sorted(_chosen(x[t], k))
    assert _close(got_ops, want), (got_ops - want).abs().max()
    assert _close(got, want), (got - want).abs().max()
    # the construction's scores are neither tiny nor all equal: every term counts
    assert want.abs().max() > 0.1


def _planted(func, old: str, new: str):
    """func with one source fragment replaced, compiled in the oracle's namespace."""
    src = textwrap.dedent(inspect.getsource(func))
    assert src.count(old) >= 1, old
    ns = dict(vars(R))
    exec(compile(src.replace(old, new), f"<planted {func.__name__}>", "exec"), ns)
    return ns[func.__name__], ns


def _swap_score_side():
    src = textwrap.dedent(inspect.getsource(R.moe_forward_reference_ops))
    assert src.count("if cfg.score_before_experts:") == 1 and src.count("if not cfg.score_before_experts:") == 1
    src = src.replace("if cfg.score_before_experts:", "if __SWAP__:")
    src = src.replace("if not cfg.score_before_experts:", "if cfg.score_before_experts:")
    src = src.replace("if __SWAP__:", "if not cfg.score_before_experts:")
    ns = dict(vars(R))
    exec(compile(src, "<planted score side>", "exec"), ns)
    return ns["moe_forward_reference_ops"]


def _token_mod_k():
    return _planted(R.moe_forward_reference_ops, "token_idx = perm // rc.top_k", "token_idx = perm % rc.top_k")[0]


def _shared_dropped():
    return _planted(R.moe_forward_reference_ops,
                    'out = feed_forward(x2, params["sw1"], params["sw2"], params["sw3"])',
                    "out = torch.zeros_like(x2)")[0]


def _score_from_choice():
    router, ns = _planted(R.router_forward_torch, "top_scores = scores.gather(dim=1, index=idx)",
                          "top_scores = choice.gather(dim=1, index=idx)")
    src = textwrap.dedent(inspect.getsource(R.moe_forward_reference_ops))
    ns["router_forward_torch"] = router
    exec(compile(src, "<planted score from choice>", "exec"), ns)
    return ns["moe_forward_reference_ops"]


PLANTED = {
    "score_on_other_side": (_swap_score_side, lambda k, sb, sh: True),
    "token_is_perm_mod_k": (_token_mod_k, lambda k, sb, sh: True),
    "shared_output_dropped": (_shared_dropped, lambda k, sb, sh: sh),
    # with one expert per token the route norm makes every score route_scale
    "score_gathered_from_biased_choice": (_score_from_choice, lambda k, sb, sh: k > 1),
}


@pytest.mark.parametrize("name", list(PLANTED))
def test_planted_glue_mistakes_fail(name):
    make, applies = PLANTED[name]
    planted = make()
    caught = 0
    for k, sb, sh in CASES:
        if not applies(k, sb, sh):
            continue
        x, p = _case(seed=10 * k + 2 * sb + sh, shared=sh)
        want = _direct(x, p, k, sb, sh)
        try:
            got = planted(p, x.view(1, N, D), _cfg(k, sb, sh)).view(N, D)
        except (IndexError, RuntimeError):
            caught += 1  # a mistake that breaks the indexing is caught as well
            continue
        assert not _close(got, want), (name, k, sb, sh)
        caught += 1
    assert caught > 0
