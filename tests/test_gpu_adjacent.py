"""GPU parity for the components adjacent to the MoE layer:

  * the aux-loss-free expert-bias update (moe_expert_bias_update) against the
    reference's own op sequence (optimizer.py:416-431, restated with the same
    torch ops in oracle.expert_bias_update) run by torch on the same GPU, and the
    optimizer step pre-hook end to end;
  * the expert-parallel local permute (moe_ep_permute_indices, gather/scatter
    rows) against the reference test's known answers (bit-exact) and the oracle
    on random counts, with permute/unpermute round trips and gradients.

Tolerance: expert_bias within 2e-9 absolute of torch's (mean(delta) sums
multiples of coeff in another order; a few ulp of coeff); everything else is
exact.
"""

import json
import os

import numpy as np
import pytest
import torch

from oracle import moe_ref as R
from tests.conftest import banner

pytestmark = pytest.mark.gpu
BIAS_TOL = 2e-9
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_bias_update_matches_reference_ops(dev):
    from torchtitan_amd.load_balancing import bias_update

    banner("expert-bias update: 5 layers, E = 256")
    gen = torch.Generator(device=dev).manual_seed(3)
    E = 256
    tpe = [torch.randint(0, 4000, (E,), generator=gen, device=dev).float() for _ in range(5)]
    tpe[1].fill_(512.0)                      # balanced: no change
    tpe[2][::4] = tpe[2].sum() / E           # values tied with the mean (when integral)
    tpe[3] = torch.zeros(E, device=dev)      # no tokens at all
    bias = [(torch.rand(E, generator=gen, device=dev) * 2 - 1) * 0.01 for _ in range(5)]
    coeffs = [1e-3, 1e-3, 5e-4, 1e-3, 1e-2]
    halve = [False, False, True, False, True]
    ref_t, ref_b = [t.clone() for t in tpe], [b.clone() for b in bias]
    R.expert_bias_update(ref_t, ref_b, coeffs, halve)
    bias_update(tpe, bias, coeffs, halve)
    torch.cuda.synchronize()
    for i in range(5):
        assert torch.count_nonzero(tpe[i]) == 0
        err = (bias[i] - ref_b[i]).abs().max().item()
        print(f"[case] layer {i}: max |bias - torch| = {err:.2e}", flush=True)
        assert err <= BIAS_TOL, (i, err)
    assert torch.equal(bias[1], ref_b[1])


def test_bias_update_hook_end_to_end(dev):
    """Two MoE layers on the GPU: a forward accumulates tokens_per_expert; the hook
    registered on a torch optimizer updates the biases before the step."""
    from torchtitan_amd import GroupedExperts, Linear, MoE, TokenChoiceTopKRouter
    from torchtitan_amd.load_balancing import register_moe_load_balancing_hook

    banner("expert-bias update through the optimizer pre-hook")

    def moe_layer():
        cfg = MoE.Config(
            num_experts=16, experts=GroupedExperts.Config(dim=256, hidden_dim=256, num_experts=16),
            router=TokenChoiceTopKRouter.Config(num_experts=16, gate=Linear.Config(in_features=256, out_features=16),
                                                top_k=2, score_func="sigmoid"),
            load_balance_coeff=1e-3)
        m = cfg.build().to(dev)
        with torch.no_grad():
            for prm in m.parameters():
                prm.data = torch.randn(prm.shape, device=dev).mul_(0.02).bfloat16()
            m.expert_bias.zero_()
            m.tokens_per_expert.zero_()
        return m

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.moe_enabled = True
            self.moe = moe_layer()

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = torch.nn.ModuleDict({"0": Block(), "1": Block()})

    torch.manual_seed(0)
    model = Model()
    x = torch.randn(2, 64, 256, device=dev).bfloat16()
    for blk in model.layers.values():
        blk.moe(x).float().sum().backward()
    before_t = [b.moe.tokens_per_expert.clone() for b in model.layers.values()]
    before_b = [b.moe.expert_bias.clone() for b in model.layers.values()]
    assert all(float(t.sum()) == 2 * 64 * 2 for t in before_t)
    R.expert_bias_update(before_t, before_b, [1e-3, 1e-3], [False, False])
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    register_moe_load_balancing_hook(opt, [model])
    opt.step()
    torch.cuda.synchronize()
    for blk, rb in zip(model.layers.values(), before_b):
        assert torch.count_nonzero(blk.moe.tokens_per_expert) == 0
        assert (blk.moe.expert_bias - rb).abs().max().item() <= BIAS_TOL


def _kats():
    with open(os.path.join(GOLDEN, "ep_permute_kats.json")) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _kats(), ids=lambda c: c["name"])
def test_ep_permute_indices_known_answers(dev, case):
    from torchtitan_amd.expert_parallel import _generate_permute_indices

    counts = torch.tensor(case["tokens_per_expert_group"], dtype=torch.int64, device=dev)
    idx, ntok = _generate_permute_indices(counts, case["experts_per_rank"], case["num_ranks"])
    ref_idx, ref_ntok = R.generate_permute_indices(case["tokens_per_expert_group"], case["experts_per_rank"],
                                                   case["num_ranks"])
    assert idx.cpu().tolist() == ref_idx.tolist()
    assert ntok.cpu().tolist() == ref_ntok.tolist()
    if case["expected_indices"] is not None:
        assert idx.cpu().tolist() == case["expected_indices"]
    if case["expected_num_tokens"] is not None:
        assert ntok.cpu().tolist() == case["expected_num_tokens"]


@pytest.mark.parametrize("ranks,experts", [(1, 8), (4, 2), (8, 16), (64, 32), (2, 1024)])
def test_ep_permute_indices_random(dev, ranks, experts):
    from torchtitan_amd.expert_parallel import _generate_permute_indices

    rng = np.random.default_rng(ranks * 1000 + experts)
    counts = rng.integers(0, 40, ranks * experts)
    counts[rng.random(counts.shape) < 0.3] = 0  # empty segments
    idx, ntok = _generate_permute_indices(torch.from_numpy(counts).to(dev), experts, ranks)
    ref_idx, ref_ntok = R.generate_permute_indices(counts, experts, ranks)
    assert np.array_equal(idx.cpu().numpy(), ref_idx) and np.array_equal(ntok.cpu().numpy(), ref_ntok)
    # a buffer longer than the received rows: the tail is marked -1
    tot = int(counts.sum())
    idx2, _ = _generate_permute_indices(torch.from_numpy(counts).to(dev), experts, ranks, total=tot + 5)
    assert np.array_equal(idx2[:tot].cpu().numpy(), ref_idx) and bool((idx2[tot:] == -1).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ep_permute_unpermute_round_trip_and_grad(dev, dtype):
    from torchtitan_amd.expert_parallel import _permute, _unpermute

    rng = np.random.default_rng(5)
    ranks, experts, d = 4, 8, 384
    counts = torch.from_numpy(rng.integers(0, 50, ranks * experts)).to(dev)
    total = int(counts.sum())
    x = torch.randn(total, d, device=dev).to(dtype).requires_grad_(True)
    shape, xp, idx, ntok = _permute(x, counts, ranks, experts)
    assert torch.equal(xp, x.detach()[idx])
    back = _unpermute(xp, shape, idx)
    assert torch.equal(back, x.detach())
    g = torch.randn(total, d, device=dev).to(dtype)
    xp.backward(g)
    xr = x.detach().clone().requires_grad_(True)
    xr[idx].backward(g)
    assert torch.equal(x.grad, xr.grad)


@pytest.mark.parametrize("pad", [16, 32])
def test_ep_permute_and_pad(dev, pad):
    """Padded expert-major layout for quantized grouped GEMMs (torchao's permute_and_pad
    as TorchAOExpertParallel calls it; torchao itself is absent, so the layout is the
    one its call site fixes): indices vs the oracle, zero padding rows, round trip."""
    from torchtitan_amd.expert_parallel import _permute_and_pad, _unpermute_padded

    rng = np.random.default_rng(pad)
    ranks, experts, d = 4, 8, 256
    counts_np = rng.integers(0, 50, ranks * experts)
    counts_np[3] = 0
    counts = torch.from_numpy(counts_np).to(dev)
    total = int(counts_np.sum())
    x = torch.randn(total, d, device=dev).bfloat16().requires_grad_(True)
    shape, xp, idx, padded, offsets = _permute_and_pad(x, counts, ranks, experts, pad)
    ref_idx, ref_padded, ref_ends = R.generate_permute_pad_indices(counts_np, experts, ranks, pad)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.array_equal(padded.cpu().numpy(), ref_padded)
    assert np.array_equal(offsets.cpu().numpy(), ref_ends)
    assert tuple(shape) == (total + 1, d)
    x_ext = torch.cat([x.detach(), torch.zeros(1, d, device=dev, dtype=x.dtype)])
    assert torch.equal(xp, x_ext[idx])
    assert torch.equal(_unpermute_padded(xp, shape, idx), x.detach())
    g = torch.randn_like(xp)
    xp.backward(g)
    xr = x_ext.clone().requires_grad_(True)
    xr[idx].backward(g)
    assert torch.equal(x.grad, xr.grad[:-1])
