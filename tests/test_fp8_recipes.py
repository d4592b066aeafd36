"""Layer-level checks that tell the fp8 recipes apart.

Rowwise fp8 (one power-of-two scale per token row, torchao's float8 grouped
GEMMs as torchtitan/components/quantization/float8.py:260-288 selects them)
and MXFP8 (one e8m0 scale per 32 elements, mx.py:85-128) quantize every element
alike except those a row scale pushes below e4m3's normal range. Random inputs
never do that, so a layer check on them cannot tell a recipe, or a scale axis,
from another. Here each token row carries a spike: its first 32 columns are
2^18 times larger than the rest, and the gate, the expert weights and the shared
expert read nothing from those columns. The row scale then maps the rest of the
row onto e4m3 subnormals (most round to 0 or +-2^-9) and the rowwise layer loses
its signal, while MX scales the spike's block alone and keeps the rest.

CPU: on the oracle's emulations the MX layer stays within 0.1 of bf16, the
rowwise layer does not, the two differ by far more than the GPU check's bound,
and so does a rowwise emulation with a planted wrong scale axis (one scale per
column of the routed rows). GPU: the fp8 and MXFP8 layers each equal their own
emulation within that bound, and differ from each other.
"""

import inspect
import textwrap

import pytest
import torch

from oracle import moe_ref as R
from tests.conftest import banner

SPIKE = 2.0 ** 18
SPIKE_COLS = 32
LAYER_TOL = 2e-2  # normwise, each layer against its own recipe's emulation
APART = 0.3       # the recipes' outputs differ by more than this


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().float(), b.detach().float()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def spike_params(p: dict) -> None:
    """Zero what reads the spike columns: the gate's, the experts' w1/w3 and the
    shared expert's w1/w3 first SPIKE_COLS input columns (in place)."""
    with torch.no_grad():
        for k in ("gate", "w1", "w3", "sw1", "sw3"):
            if k in p:
                p[k][..., :SPIKE_COLS] = 0


def spike_x(x: torch.Tensor, gen: torch.Generator) -> torch.Tensor:
    x = x.clone()
    big = torch.randn(x.shape[:-1] + (SPIKE_COLS,), generator=gen, device=x.device) * SPIKE
    x[..., :SPIKE_COLS] = big.to(x.dtype)
    return x


def _cfg(kind: str, e: int, k: int, d: int, h: int) -> R.MoECfg:
    rc = R.RouterCfg(num_experts=e, top_k=k, score_func="sigmoid", route_norm=True, route_scale=2.5)
    return R.MoECfg(router=rc, dim=d, hidden_dim=h, score_before_experts=True, use_grouped_mm=True,
                    has_shared=False, expert_kind=kind)


def _cpu_case(seed=3, n=256, d=128, e=4, k=2, h=64):
    g = torch.Generator().manual_seed(seed)
    p = {"gate": (torch.randn(e, d, generator=g) * 0.05).bfloat16(),
         "expert_bias": (torch.rand(e, generator=g) * 2 - 1) * 0.01,
         "w1": (torch.randn(e, h, d, generator=g) * 0.05).bfloat16(),
         "w2": (torch.randn(e, d, h, generator=g) * 0.05).bfloat16(),
         "w3": (torch.randn(e, h, d, generator=g) * 0.05).bfloat16()}
    spike_params(p)
    x = spike_x(torch.randn(1, n, d, generator=g).bfloat16(), g)
    return p, x, (e, k, d, h)


def _planted_rowwise_wrong_axis():
    """experts_fp8_forward with x scaled per column of the routed rows."""
    src = textwrap.dedent(inspect.getsource(R.experts_fp8_forward))
    old = "qx, sx = quant_fp8_rows(x)"
    assert src.count(old) == 1
    ns = dict(vars(R))
    # one scale per column; the column scales are applied before the product
    new = "qx, sx = quant_fp8_rows(x, dim=0); qx, sx = qx.double() * sx.double(), torch.ones(x.shape[0], 1)"
    exec(compile(src.replace(old, new), "<planted axis>", "exec"), ns)
    lsrc = textwrap.dedent(inspect.getsource(R.moe_forward_reference_ops))
    exec(compile(lsrc, "<layer with planted axis>", "exec"), ns)
    return ns["moe_forward_reference_ops"]


def test_recipes_apart_on_spiked_rows_cpu():
    p, x, (e, k, d, h) = _cpu_case()
    out_bf = R.moe_forward_reference_ops(p, x, _cfg("swiglu", e, k, d, h))
    out_f8 = R.moe_forward_reference_ops(p, x, _cfg("fp8", e, k, d, h))
    out_mx = R.moe_forward_reference_ops(p, x, _cfg("mxfp8", e, k, d, h))
    assert rel(out_mx, out_bf) <= 0.1
    assert rel(out_f8, out_bf) > APART
    assert rel(out_f8, out_mx) > APART
    planted = _planted_rowwise_wrong_axis()(p, x, _cfg("fp8", e, k, d, h))
    # the planted axis keeps the signal: it fails the rowwise layer check by far
    assert rel(planted, out_f8) > 10 * LAYER_TOL
    assert rel(planted, out_bf) <= 0.1


def test_recipes_agree_without_spikes_cpu():
    """Without the spike both recipes track bf16 and each other (which is why a
    random-input layer check cannot tell them apart)."""
    p, x, (e, k, d, h) = _cpu_case()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(x.shape, generator=g).bfloat16()
    out_bf = R.moe_forward_reference_ops(p, x, _cfg("swiglu", e, k, d, h))
    out_f8 = R.moe_forward_reference_ops(p, x, _cfg("fp8", e, k, d, h))
    out_mx = R.moe_forward_reference_ops(p, x, _cfg("mxfp8", e, k, d, h))
    assert rel(out_f8, out_bf) <= 0.1 and rel(out_mx, out_bf) <= 0.1 and rel(out_f8, out_mx) <= 0.1


GPU_SHAPE = dict(bs=2, slen=2048, dim=1024, experts=16, top_k=4, hidden=512, shared_hidden=0)


@pytest.mark.gpu
def test_fp8_and_mxfp8_layers_follow_their_recipe_on_spiked_rows(dev):
    from tests.layer_util import LayerShape, build_layer

    banner("fp8 / MXFP8 layers on spiked rows against their emulations")
    outs = {}
    for kind in ("bf16", "fp8", "mxfp8"):
        sh = LayerShape(**GPU_SHAPE, fp8=kind == "fp8", mxfp8=kind == "mxfp8")
        moe, x, _ = build_layer(sh, dev, seed=21)  # the same weights and x for every kind
        sd = moe.state_dict()
        p = {"gate": moe.router.gate.weight.data, "w1": moe.experts.w1.data, "w3": moe.experts.w3.data}
        spike_params(p)
        xs = spike_x(x, torch.Generator(device=dev).manual_seed(22))
        with torch.no_grad():
            outs[kind] = moe(xs).float()
        params = {"gate": sd["router.gate.weight"], "w1": sd["experts.w1"], "w2": sd["experts.w2"],
                  "w3": sd["experts.w3"], "expert_bias": sd["expert_bias"]}
        if kind != "bf16":
            cfg = _cfg(kind, sh.experts, sh.top_k, sh.dim, sh.hidden)
            with torch.no_grad():
                emu = R.moe_forward_reference_ops(params, xs, cfg).float()
            err = rel(outs[kind], emu)
            print(f"[case] {kind}: layer vs its emulation {err:.2e}", flush=True)
            assert err <= LAYER_TOL, (kind, err)
        del moe
    d_f8, d_mx, d_apart = rel(outs["fp8"], outs["bf16"]), rel(outs["mxfp8"], outs["bf16"]), rel(outs["fp8"],
                                                                                                  outs["mxfp8"])
    print(f"[case] vs bf16: fp8 {d_f8:.2e}, mxfp8 {d_mx:.2e}; fp8 vs mxfp8 {d_apart:.2e}", flush=True)
    assert d_mx <= 0.1
    assert d_f8 > APART and d_apart > APART
