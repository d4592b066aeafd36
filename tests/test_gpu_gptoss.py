"""gpt-oss experts (torchtitan/models/gpt_oss/moe.py:43-122) on the GPU.

The layer's op (ops.grouped_swiglu_oss: the bf16 grouped GEMMs with the
biased, clamped SwiGLU epilogues) against the reference's own grouped-mm op
sequence (oracle.oss_experts_grouped_mm: torch._grouped_mm, repeat_interleave
biases, the torch swiglu) run by torch on the same GPU, forward and autograd.
Weights are bf16, biases fp32 (as master weights; the reference then sums the
bias gradients in fp32). Shapes include gpt-oss's D = H = 2880, which leaves
partial tiles, and weight scales that drive a large share of h1 past the clamp
limit. Tolerance: 1e-2 normwise relative error (max |ours - ref| / max |ref|)
for every output and gradient; the bias gradients are also checked against
fp64 sums of our own dh1 / dy rows (the fixed-order column-sum kernel).
"""

import pytest
import torch

from oracle import moe_ref as R
from tests.conftest import banner

pytestmark = pytest.mark.gpu

TOL = 1e-2

CASES = {
    "e8_d256_h320": (8, 256, 320, [100, 0, 257, 31, 64, 200, 1, 90], 7.0),
    "gptoss_dims_e4": (4, 2880, 2880, [300, 0, 513, 77], 7.0),
    "limit_2_5": (4, 512, 256, [64, 129, 0, 40], 2.5),
}


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("name", list(CASES))
def test_oss_experts_match_reference_ops_on_device(dev, name):
    e, d, h, counts, limit = CASES[name]
    banner(f"gpt-oss experts {name}")
    from torchtitan_amd import gpt_oss

    g = torch.Generator().manual_seed(11)
    r = sum(counts)
    cnt = torch.tensor(counts, dtype=torch.int64, device=dev)
    x = torch.randn(r, d, generator=g).bfloat16().to(dev)
    w1 = (torch.randn(e, 2 * h, d, generator=g) * (6.0 / d ** 0.5)).bfloat16().to(dev)
    b1 = (torch.randn(e, 2 * h, generator=g) * 0.5).to(dev)
    w2 = (torch.randn(e, d, h, generator=g) * (1.0 / h ** 0.5)).bfloat16().to(dev)
    b2 = (torch.randn(e, d, generator=g) * 0.5).to(dev)
    dy = torch.randn(r, d, generator=g).bfloat16().to(dev)

    ours = [t.clone().requires_grad_(True) for t in (x, w1, b1, w2, b2)]
    y = gpt_oss._run_experts_grouped_mm(ours[1], ours[2], ours[3], ours[4], limit, ours[0], cnt)
    y.backward(dy)
    ref = [t.clone().requires_grad_(True) for t in (x, w1, b1, w2, b2)]
    yr = R.oss_experts_grouped_mm(ref[1], ref[2], ref[3], ref[4], limit, ref[0], cnt)
    yr.backward(dy)
    torch.cuda.synchronize()

    # share of the glu / linear inputs beyond the clamp (the reference's h1 before swiglu)
    with torch.no_grad():
        h1 = torch._grouped_mm(x, w1.transpose(-2, -1), offs=torch.cumsum(cnt, 0, dtype=torch.int32))
        clamped = ((h1[:, ::2] > limit).float().mean().item(), (h1[:, 1::2].abs() > limit).float().mean().item())
    errs = {"y": _rel(y, yr), "dx": _rel(ours[0].grad, ref[0].grad), "dmlp1": _rel(ours[1].grad, ref[1].grad),
            "dmlp1_bias": _rel(ours[2].grad, ref[2].grad), "dmlp2": _rel(ours[3].grad, ref[3].grad),
            "dmlp2_bias": _rel(ours[4].grad, ref[4].grad)}
    same = {"y": (y == yr).float().mean().item(), "dx": (ours[0].grad == ref[0].grad).float().mean().item()}
    print(f"[case] {name}: clamped glu {clamped[0]:.2f} linear {clamped[1]:.2f}; errs {errs}; "
          f"bit-identical fraction {same}", flush=True)
    assert clamped[0] > 0.05 and clamped[1] > 0.05
    assert all(v <= TOL for v in errs.values()), errs
    for i, c in enumerate(counts):
        if c == 0:
            for t in (ours[1].grad, ours[2].grad, ours[3].grad, ours[4].grad):
                assert torch.count_nonzero(t[i]) == 0


def test_grouped_col_sum_exact_order(dev):
    banner("grouped column sums")
    from torchtitan_amd import _lib

    g = torch.Generator().manual_seed(2)
    counts = [0, 5, 1000, 33, 0, 257]
    r, c = sum(counts), 192
    src = torch.randn(r, 2 * c, generator=g).bfloat16()
    cnt = torch.tensor(counts, dtype=torch.int64)
    sd, cd = src.to(dev), cnt.to(dev)
    out = torch.full((len(counts), 2 * c), float("nan"), device=dev)
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("moe_grouped_col_sum", sd.data_ptr(), 2 * c, cd.data_ptr(), r, len(counts), c, out.data_ptr(), 2 * c, 2,
              st)
    _lib.call("moe_grouped_col_sum", sd.data_ptr() + 2 * c, 2 * c, cd.data_ptr(), r, len(counts), c,
              out.data_ptr() + 4, 2 * c, 2, st)
    torch.cuda.synchronize()
    ref, s0 = torch.zeros(len(counts), 2 * c, dtype=torch.float64), 0
    for i, n in enumerate(counts):
        seg = src[s0:s0 + n].double()
        ref[i, 0::2] = seg[:, :c].sum(0)
        ref[i, 1::2] = seg[:, c:].sum(0)
        s0 += n
    o = out.cpu().double()
    assert torch.isfinite(o).all()
    assert ((o - ref).abs() <= 1e-5 * ref.abs().clamp_min(1.0)).all()
    assert torch.count_nonzero(o[0]) == 0 and torch.count_nonzero(o[4]) == 0
