"""The shared expert (torchtitan/models/common/feed_forward.py:34-54) on the GPU
against the reference's own module (three nn.Linear and autograd) with the same
bf16 parameters and inputs:
  * output and input gradient bit-identical (the same library calls);
  * weight gradients compared with the fp64 product of the exact bf16 operands
    each weight-gradient GEMM consumes: every element within the error bound of
    an fp32 accumulation in any order followed by one rounding to bf16,
    |dW - T| <= n 2^-24 (|A|^T |B|) + ulp_bf16(|T| + n 2^-24 (|A|^T |B|)) / 2,
    which the reference's GEMM meets too, and differing from bf16(T) in at most
    1e-3 more of the elements than the reference's do.
"""

import pytest
import torch
import torch.nn.functional as F

from tests.conftest import banner
from torchtitan_amd import FeedForward, Linear

pytestmark = pytest.mark.gpu

CASES = {
    "kimi_n16384_d2304_h1024": (16384, 2304, 1024),
    "dsv3_n8192_d7168_h2048": (8192, 7168, 2048),
    "unsplit_n3000_d256_h512": (3000, 256, 512),
}


def _ulp_bf16(t: torch.Tensor) -> torch.Tensor:
    e = torch.floor(torch.log2(t.abs().clamp_min(2.0 ** -126)))
    return torch.exp2(e - 7)


@pytest.mark.parametrize("case", list(CASES))
def test_shared_expert_matches_reference_module(dev, case):
    n, d, h = CASES[case]
    banner(f"shared expert {case}")
    g = torch.Generator(device=dev).manual_seed(3)
    ff = FeedForward(FeedForward.Config(w1=Linear.Config(in_features=d, out_features=h),
                                        w2=Linear.Config(in_features=h, out_features=d),
                                        w3=Linear.Config(in_features=d, out_features=h))).to(dev)
    ref = [torch.nn.Linear(d, h, bias=False), torch.nn.Linear(h, d, bias=False), torch.nn.Linear(d, h, bias=False)]
    with torch.no_grad():
        for lin, r in zip((ff.w1, ff.w2, ff.w3), ref):
            lin.weight.data = (torch.randn(lin.weight.shape, generator=g, device=dev) * 0.02).bfloat16()
            r.to(dev)
            r.weight.data = lin.weight.data.clone()
    x = torch.randn(2, n // 2, d, generator=g, device=dev).bfloat16()
    gy = torch.randn(2, n // 2, d, generator=g, device=dev).bfloat16()

    xa = x.clone().requires_grad_(True)
    out = ff(xa)
    out.backward(gy)
    xb = x.clone().requires_grad_(True)
    r1, r2, r3 = ref
    a1, a3 = r1(xb), r3(xb)
    hh = F.silu(a1) * a3
    for t in (a1, a3, hh):
        t.retain_grad()
    out_r = r2(hh)
    out_r.backward(gy)
    torch.cuda.synchronize()
    assert torch.equal(out, out_r), "output differs from the reference module"
    assert torch.equal(xa.grad, xb.grad), "input gradient differs from the reference module"

    # fp64 products of the exact bf16 operands each weight-gradient GEMM consumes
    with torch.no_grad():
        x2, gy2 = x.reshape(n, d).double(), gy.reshape(n, d).double()
        ops = {"w2": (gy2, hh.reshape(n, h).double()),
               "w1": (a1.grad.reshape(n, h).double(), x2),
               "w3": (a3.grad.reshape(n, h).double(), x2)}
    gamma = n * 2.0 ** -24
    for name, lin, r in (("w1", ff.w1, r1), ("w2", ff.w2, r2), ("w3", ff.w3, r3)):
        a, b = ops[name]
        truth = (a.t() @ b).float()
        bound = gamma * (a.abs().t() @ b.abs()).float()
        bound = bound + 0.5 * _ulp_bf16(truth.abs() + bound)
        tb = truth.bfloat16().float()
        ours, theirs = lin.weight.grad.float(), r.weight.grad.float()
        ratio_o = ((ours - truth).abs() / bound).max().item()
        ratio_r = ((theirs - truth).abs() / bound).max().item()
        frac_o = (ours != tb).float().mean().item()
        frac_r = (theirs != tb).float().mean().item()
        print(f"[case] {case} d{name}: max error / bound ours {ratio_o:.3f} ref {ratio_r:.3f}; "
              f"elements != bf16(fp64) ours {frac_o:.2e} ref {frac_r:.2e}", flush=True)
        assert ratio_o <= 1.0
        assert frac_o <= frac_r + 1e-3


SWIGLU_CASES = {
    # rows, Hs, dtype, element offset of the views (0: 16-byte aligned)
    "bf16_kimi": (16384, 1024, torch.bfloat16, 0),
    "bf16_width_1000": (257, 1000, torch.bfloat16, 0),
    "bf16_width_97_scalar": (300, 97, torch.bfloat16, 0),
    "bf16_misaligned": (64, 256, torch.bfloat16, 3),
    "fp32_512": (333, 512, torch.float32, 0),
    "fp32_width_30_scalar": (100, 30, torch.float32, 0),
}


@pytest.mark.parametrize("case", list(SWIGLU_CASES))
def test_swiglu_kernels_match_torch_ops_and_autograd(dev, case):
    """ops.swiglu_forward is torch's silu(a1) * a3 and ops.swiglu_backward its
    autograd (silu_backward(dh * a3, a1) | dh * silu(a1)) bit for bit, run by torch
    on the same device; widths off the 16-byte chunk and misaligned views take the
    one-element-per-thread kernels."""
    from torchtitan_amd import ops

    rows, hs, dt, off = SWIGLU_CASES[case]
    banner(f"swiglu kernels {case}")
    g = torch.Generator(device=dev).manual_seed(11)

    def t(scale):
        base = (torch.randn(rows * hs + off, generator=g, device=dev) * scale).to(dt)
        return base[off:].view(rows, hs)

    a1, a3, dh = t(3.0), t(1.0), t(0.5)
    a1[0, : min(hs, 4)] = torch.tensor([0.0, -0.0, 30.0, -30.0][: min(hs, 4)], device=dev).to(dt)
    h = ops.swiglu_forward(a1, a3)
    assert torch.equal(h, F.silu(a1) * a3)
    ra1, ra3 = a1.clone().requires_grad_(True), a3.clone().requires_grad_(True)
    (F.silu(ra1) * ra3).backward(dh)
    dgu = ops.swiglu_backward(dh, a1, a3)
    assert dgu.shape == (rows, 2 * hs)
    assert torch.equal(dgu[:, :hs], ra1.grad)
    assert torch.equal(dgu[:, hs:], ra3.grad)


def test_swiglu_kernels_every_bf16(dev):
    """The shared expert's SwiGLU kernels on a1 covering every bf16 value (the values
    where they divide in the reciprocal form in rows 0-207, the rest after): h, dg
    and du equal torch's ops and autograd bit for bit, NaNs as NaNs."""
    from tests.test_gpu_kernels import _bf16_patterns_split, _fill_rows
    from torchtitan_amd import ops

    banner("swiglu kernels, every bf16 a1")
    hs = 256
    fast, rest = _bf16_patterns_split()
    a1 = torch.cat([_fill_rows(fast, 208, hs), _fill_rows(rest, 112, hs)]).to(dev)
    g = torch.Generator().manual_seed(5)
    a3 = (torch.randn(a1.shape, generator=g) * 2).bfloat16().to(dev)
    dh = (torch.randn(a1.shape, generator=g) * 2).bfloat16().to(dev)

    def same(a, b):
        return bool(((a.view(torch.int16) == b.view(torch.int16)) | (torch.isnan(a) & torch.isnan(b))).all())

    assert same(ops.swiglu_forward(a1, a3), F.silu(a1) * a3)
    ra1, ra3 = a1.clone().requires_grad_(True), a3.clone().requires_grad_(True)
    (F.silu(ra1) * ra3).backward(dh)
    dgu = ops.swiglu_backward(dh, a1, a3)
    assert same(dgu[:, :hs], ra1.grad)
    assert same(dgu[:, hs:], ra3.grad)
