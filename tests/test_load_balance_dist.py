"""The expert-bias update across ranks, on the CPU with gloo (world size 2).

The reference floors each rank's double-counted tokens (activation
checkpointing) before it sums the counts over the loss mesh
(torchtitan/components/optimizer.py:389-394, then :400-414). The hook must do
the same: with odd counts on both ranks, flooring after the sum gives another
result. The kernel launch itself (GPU only) is replaced by a recorder here.
"""

import os
import socket

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _worker(rank: int, world: int, port: int, queue) -> None:
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        from torch.distributed.algorithms._checkpoint.checkpoint_wrapper import CheckpointImpl

        from torchtitan_amd import load_balancing as LB
        from tests.test_modules import _cfg

        class Block(torch.nn.Module):
            def __init__(self, recompute: bool):
                super().__init__()
                self.moe_enabled = True
                self.moe = _cfg(hs=0, coeff=1e-3).build()
                if recompute:
                    self.checkpoint_impl = CheckpointImpl.NO_REENTRANT

        class Model(torch.nn.Module):
            def __init__(self):
                super().__init__()
                self.layers = torch.nn.ModuleDict({"0": Block(True), "1": Block(False)})

        model = Model()
        e = model.layers["0"].moe.tokens_per_expert.numel()
        # odd counts on every rank: 2r + 1 + expert index
        for blk in model.layers.values():
            blk.moe.tokens_per_expert.copy_(torch.arange(e, dtype=torch.float32) + 2 * rank + 1)
        seen = {}

        def record(tpe, bias, coeffs, halve):
            seen["tpe"] = [t.clone() for t in tpe]
            seen["halve"] = list(halve)

        LB.bias_update = record
        LB.update_expert_bias([model], group=dist.group.WORLD)
        queue.put((rank, [t.tolist() for t in seen["tpe"]], seen["halve"]))
    finally:
        dist.destroy_process_group()


def test_halving_floors_per_rank_before_the_sum():
    world = 2
    ctx = mp.get_context("spawn")
    queue = ctx.Queue()
    port = _free_port()
    procs = [ctx.Process(target=_worker, args=(r, world, port, queue)) for r in range(world)]
    for p in procs:
        p.start()
    results = [queue.get(timeout=120) for _ in range(world)]
    for p in procs:
        p.join(timeout=60)
        assert p.exitcode == 0
    e = len(results[0][1][0])
    base = [torch.arange(e, dtype=torch.float32) + 2 * r + 1 for r in range(world)]
    per_rank_floor = sum(torch.floor(b / 2) for b in base)  # the reference's order
    floor_of_sum = torch.floor(sum(base) / 2)
    assert not torch.equal(per_rank_floor, floor_of_sum)  # the case tells the two orders apart
    for _rank, tpe, halve in results:
        assert halve == [False, False]  # already halved before the all-reduce
        assert torch.equal(torch.tensor(tpe[0]), per_rank_floor)  # recomputed block
        assert torch.equal(torch.tensor(tpe[1]), sum(base))  # plain block: the plain sum


if __name__ == "__main__":
    pytest.main([__file__, "-q"])
