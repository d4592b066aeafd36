"""Graph capture of the bf16 MoE layer's forward + backward.

The path has no host synchronisation: the router, the reorder, the persistent
grouped GEMMs (which read the per-expert counts on the device) and the combine
take every size from device memory, so one captured graph serves any routing.
The Kimi-Linear-48B-shape layer (16384 tokens, dim 2304, 256 experts top-8,
hidden 1024, shared expert) is captured with torch.cuda.graph and replayed
several times, on the captured input and on a second input copied into the
same buffer (another routing, other per-expert counts), with eager layer calls
and synchronisations between the replays; every replay's output, input
gradient and parameter gradients equal the eager run on the same input bit for
bit. (The reference cannot capture this path: its graph trainer refuses
torch._grouped_mm, torchtitan/experiments/graph_trainer/cudagraph.py:243-245.)
"""

import pytest
import torch

from tests.conftest import banner

pytestmark = pytest.mark.gpu

KIMI = dict(bs=4, slen=4096, dim=2304, experts=256, top_k=8, hidden=1024, shared_hidden=1024)


def test_layer_forward_backward_graph_replays_equal_eager(dev):
    from tests.layer_util import LayerShape, build_layer

    banner("graph capture of the Kimi-shape bf16 layer fwd+bwd")
    sh = LayerShape(**KIMI)
    moe, x1, gy = build_layer(sh, dev, seed=11)
    x2 = torch.randn(x1.shape, device=dev, generator=torch.Generator(device=dev).manual_seed(12)).to(x1.dtype)
    params = [p for p in moe.parameters() if p.requires_grad]

    def step(xin):
        out = moe(xin)
        out.backward(gy)
        return out

    def eager(xv):
        xe = xv.clone().requires_grad_(True)
        moe.zero_grad(set_to_none=True)
        out = step(xe)
        torch.cuda.synchronize()
        return out.detach().clone(), xe.grad.clone(), [p.grad.clone() for p in params]

    ref = {1: eager(x1), 2: eager(x2)}
    assert not torch.equal(ref[1][0], ref[2][0])

    static_x = x1.clone().requires_grad_(True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):  # warm-up on a side stream before capture
            moe.zero_grad(set_to_none=True)
            static_x.grad = None
            step(static_x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    moe.zero_grad(set_to_none=True)
    static_x.grad = None
    graph = torch.cuda.CUDAGraph()
    banner("capturing")
    with torch.cuda.graph(graph):
        static_out = step(static_x)
    static_gx = static_x.grad
    static_gp = [p.grad for p in params]

    for i, which in enumerate((1, 1, 2, 1, 2)):
        banner(f"replay {i} on input {which}")
        with torch.no_grad():
            static_x.copy_(x1 if which == 1 else x2)
        graph.replay()
        torch.cuda.synchronize()
        out, gx, gp = ref[which]
        assert torch.equal(static_out, out), f"replay {i}: output"
        assert torch.equal(static_gx, gx), f"replay {i}: grad_x"
        for j, (a, b) in enumerate(zip(static_gp, gp)):
            assert torch.equal(a, b), f"replay {i}: parameter gradient {j}"
        # the program's own eager work between replays
        with torch.no_grad():
            moe(x2 if which == 1 else x1)
        torch.cuda.synchronize()
    del graph
