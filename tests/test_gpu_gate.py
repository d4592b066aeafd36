"""Router gate logits in fp32 (torchtitan/models/common/moe.py:230-232) on the GPU.

The layer's default gate computes its logits with the reference's own call (the
fp32 GEMM under autocast), which the tests below check bit for bit, and its
backward on bf16 GEMMs over an exact three-term split of the fp32 logit
gradient (moe._GateRef). That backward, the opt-in gate (``bf16_mfma=True``:
forward too on bf16 GEMMs with fp32 accumulation, moe._GateF32) and the fp32
autocast path are checked against the fp64 product of the same values:
  * logits: the error of the bf16-GEMM path is at most 2x the fp32 path's
    (plus 1e-6 of the largest logit): both are fp32 sums of the same exact
    products, in different orders;
  * dx, dW (rounded to bf16): equal to bf16(fp64 gradient) wherever the fp32
    path is, except at most 1e-3 of the elements, which may sit on a bf16
    rounding boundary; the worst error, in bf16 ulps of the true value, at
    most twice the fp32 path's (where the sum cancels to a value far below its
    terms both are many ulps off) or one ulp;
  * bias gradient: the fp32 column sum of the logit gradient.
The upstream gradient spans six decades, so the second and third bf16 terms of
its split carry weight. The opt-in gate's logits are the fp32 GEMM's to
summation order only, so a token whose K-th and (K+1)-th biased scores nearly
tie can get another expert set: test_opt_in_gate_routing_disagreement counts
how often at the Kimi-Linear layer shapes.
"""

import pytest
import torch
import torch.nn.functional as F

from tests.conftest import banner
from torchtitan_amd import Linear
from torchtitan_amd.moe import gate_logits_f32

pytestmark = pytest.mark.gpu

CASES = {
    "kimi_dim2304_e256": (4096, 2304, 256, False),
    "gptoss_dim2880_e32_bias": (2048, 2880, 32, True),
    "ragged_n1000_dim768_e64": (1000, 768, 64, False),
}


def _ulp_bf16(t: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values around |t| (fp32 tensor)."""
    e = torch.floor(torch.log2(t.abs().clamp_min(2.0 ** -126)))
    return torch.exp2(e - 7)


@pytest.mark.parametrize("mode", ["default", "bf16_mfma"])
@pytest.mark.parametrize("case", list(CASES))
def test_gate_logits_f32_vs_fp64(case, mode):
    n, d, e, bias = CASES[case]
    banner(f"gate {case} {mode}: n={n} dim={d} experts={e} bias={bias}")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    gate = Linear(Linear.Config(in_features=d, out_features=e, bias=bias)).to(dev)
    with torch.no_grad():
        gate.weight.data = (torch.randn(e, d, generator=g, device=dev) * 0.02).bfloat16()
        if bias:
            gate.bias.data = (torch.randn(e, generator=g, device=dev) * 0.1).bfloat16()
    x = torch.randn(n, d, generator=g, device=dev).bfloat16()
    mag = torch.exp(torch.empty(n, e, device=dev).uniform_(-7.0, 7.0, generator=g))
    up = torch.randn(n, e, generator=g, device=dev) * mag

    def run(fast: bool):
        xs = x.clone().requires_grad_(True)
        gate.zero_grad(set_to_none=True)
        if fast:
            y = gate_logits_f32(xs, gate, bf16_mfma=(mode == "bf16_mfma"))
        else:
            with torch.autocast(device_type="cuda", dtype=torch.float32):
                y = gate(xs)
        y.backward(up)
        return y.detach(), xs.grad, gate.weight.grad, gate.bias.grad if bias else None

    y_f, dx_f, dw_f, db_f = run(True)
    y_r, dx_r, dw_r, db_r = run(False)
    assert y_f.dtype == torch.float32 and dx_f.dtype == torch.bfloat16 and dw_f.dtype == torch.bfloat16

    xd, wd, upd = x.double(), gate.weight.detach().double(), up.double()
    y_t = xd @ wd.t()
    if bias:
        y_t = y_t + gate.bias.detach().double()
    err_f = (y_f.double() - y_t).abs().max().item()
    err_r = (y_r.double() - y_t).abs().max().item()
    scale = y_t.abs().max().item()
    print(f"[case] {case}: logits max err fast {err_f:.3e} fp32-autocast {err_r:.3e} (max |logit| {scale:.3e})",
          flush=True)
    assert err_f <= 2 * err_r + 1e-6 * scale
    if mode == "default":
        assert torch.equal(y_f, y_r), "the default gate's logits are not the autocast GEMM's bits"

    for name, got, ref, truth in (
        ("dx", dx_f, dx_r, upd @ wd),
        ("dW", dw_f, dw_r, upd.t() @ xd),
    ):
        t32 = truth.float()
        tb = t32.bfloat16().float()
        diff_f = (got.float() != tb)
        diff_r = (ref.float() != tb)
        frac_f = diff_f.float().mean().item()
        frac_r = diff_r.float().mean().item()
        worst_f = ((got.float() - t32).abs() / _ulp_bf16(t32)).max().item()
        worst_r = ((ref.float() - t32).abs() / _ulp_bf16(t32)).max().item()
        print(f"[case] {case}: {name} elements != bf16(fp64): fast {frac_f:.2e} fp32-autocast {frac_r:.2e}; "
              f"worst ulp fast {worst_f:.2f} fp32-autocast {worst_r:.2f}", flush=True)
        assert frac_f <= frac_r + 1e-3
        assert worst_f <= max(1.0, 2 * worst_r)
    if bias:
        assert torch.allclose(db_f.float(), upd.sum(0).float(), rtol=1e-2, atol=0)
        assert torch.equal(db_f, db_r) or (db_f.float() - db_r.float()).abs().max() <= _ulp_bf16(
            upd.sum(0).float()).max()


def test_gate_logits_fallback_paths():
    """The default gate is the reference's autocast region for bf16 weights; fp32
    weights, or an outer autocast, keep it also when the opt-in is asked for."""
    dev = torch.device("cuda:0")
    gate = Linear(Linear.Config(in_features=256, out_features=16)).to(dev)
    x = torch.randn(64, 256, device=dev).bfloat16()
    gb = Linear(Linear.Config(in_features=256, out_features=16)).to(dev)
    gb.weight.data = gb.weight.data.bfloat16()
    with torch.autocast(device_type="cuda", dtype=torch.float32):
        ref0 = gb(x)
    assert torch.equal(gate_logits_f32(x, gb), ref0)  # default: the reference's call
    y = gate_logits_f32(x, gate, bf16_mfma=True)  # fp32 weight
    with torch.autocast(device_type="cuda", dtype=torch.float32):
        ref = gate(x)
    assert torch.equal(y, ref)
    gate.weight.data = gate.weight.data.bfloat16()
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        y2 = gate_logits_f32(x, gate, bf16_mfma=True)
    with torch.autocast(device_type="cuda", dtype=torch.float32):
        ref2 = F.linear(x, gate.weight)
    assert y2.dtype == torch.float32 and torch.equal(y2, ref2)


@pytest.mark.parametrize("n_tokens,zipf", [(16384, False), (32768, True)])
def test_opt_in_gate_routing_disagreement(n_tokens, zipf):
    """How often the opt-in bf16-MFMA gate routes a token to another expert set
    than the reference's fp32 autocast gate, at the Kimi-Linear layer shape (dim
    2304, 256 experts, top-8 sigmoid + expert bias), over three seeds. The
    default gate is the reference's call and never disagrees; the rate of the
    opt-in one is printed and bounded at 1e-3 of the tokens."""
    from oracle import moe_ref as R

    dev = torch.device("cuda:0")
    d, e, k = 2304, 256, 8
    rc = R.RouterCfg(num_experts=e, top_k=k, score_func="sigmoid", route_norm=True, route_scale=2.5)
    total, differ = 0, 0
    for seed in (1, 2, 3):
        banner(f"opt-in gate routing n={n_tokens} zipf={zipf} seed={seed}")
        g = torch.Generator(device=dev).manual_seed(seed)
        gate = Linear(Linear.Config(in_features=d, out_features=e)).to(dev)
        gate.weight.data = (torch.randn(e, d, generator=g, device=dev) * 0.02).bfloat16()
        bias = (torch.rand(e, generator=g, device=dev) * 2 - 1) * 0.01
        if zipf:
            ranks = torch.randperm(e, generator=g, device=dev).float() + 1.0
            bias = bias + 0.25 * ranks.pow(-1.2) - 1.0 * (ranks > e - 20).float()
        x = torch.randn(n_tokens, d, generator=g, device=dev).bfloat16()
        with torch.no_grad():
            ref = gate_logits_f32(x, gate)
            fast = gate_logits_f32(x, gate, bf16_mfma=True)
            _, i_ref, _, _ = R.router_forward_torch(ref, bias, rc)
            _, i_fast, _, _ = R.router_forward_torch(fast, bias, rc)
        s_ref = torch.sort(i_ref, dim=1).values
        s_fast = torch.sort(i_fast, dim=1).values
        differ += int((s_ref != s_fast).any(dim=1).sum())
        total += n_tokens
    rate = differ / total
    print(f"[case] opt-in gate: {differ} of {total} tokens routed to another expert set ({rate:.2e})",
          flush=True)
    assert rate <= 1e-3


@pytest.mark.parametrize("shape", [(16384, 256), (1000, 64), (3, 8)])
def test_gate_grad_split3_kernel_matches_torch_casts(shape):
    """ops.gate_grad_split3 equals the three torch casts and subtractions of the
    oracle run on the device, bit for bit, over twelve decades of magnitude,
    signed zeros, infinities and NaN; the terms add back to the gradient."""
    from oracle.moe_ref import gate_grad_split3
    from torchtitan_amd import ops

    n, e = shape
    banner(f"gate split3 {n}x{e}")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    d = torch.randn(n, e, generator=g, device=dev) * torch.exp(
        torch.empty(n, e, device=dev).uniform_(-14.0, 14.0, generator=g))
    d[0, :4] = torch.tensor([0.0, -0.0, float("inf"), float("nan")], device=dev)
    got = ops.gate_grad_split3(d)
    want = gate_grad_split3(d)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    fin = torch.isfinite(d)
    hi, mid, lo = (got[:, i * e:(i + 1) * e].float() for i in range(3))
    assert torch.equal(((hi + mid) + lo)[fin], d[fin])


@pytest.mark.parametrize("parts", [1, 2])
@pytest.mark.parametrize("e_d", [(256, 2304), (8, 256)])
def test_gate_dw_reduce_kernel_matches_torch_adds(parts, e_d):
    """ops.gate_dw_reduce equals the oracle's fp32 adds ((halves), then
    (hi + mid) + lo) and bf16 cast run on the device, bit for bit."""
    from oracle.moe_ref import gate_dw_reduce
    from torchtitan_amd import ops

    e, d = e_d
    banner(f"gate dw reduce parts={parts} e={e} d={d}")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(9)
    shape = (parts, 3 * e, d) if parts == 2 else (3 * e, d)
    p = torch.randn(*shape, generator=g, device=dev) * torch.exp(
        torch.empty(*shape, device=dev).uniform_(-8.0, 8.0, generator=g))
    assert torch.equal(ops.gate_dw_reduce(p, e).view(torch.int16), gate_dw_reduce(p, e).view(torch.int16))
