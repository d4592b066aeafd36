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
