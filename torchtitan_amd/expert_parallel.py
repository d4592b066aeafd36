"""Expert-parallel local permute on the MI355X kernels.

Mirrors torchtitan/distributed/expert_parallel.py:26-80: after the token
all-to-all, a rank holds segments of rows in rank-major order (source rank r,
local expert e); the grouped GEMMs need them expert-major. The index generation
and both row movements run as HIP kernels (``moe_ep_permute_indices``,
``moe_gather_rows``, ``moe_scatter_rows``). The all-to-all itself is RCCL's and
is not part of this one-GPU build.
"""

from __future__ import annotations

import torch

from . import ops
from ._lib import call, ptr, require_gpu, stream_of


def _generate_permute_indices(tokens_per_expert_group: torch.Tensor, experts_per_rank: int, num_ranks: int,
                              total: int | None = None):
    """Returns (permuted_indices [total] int64, num_tokens_per_expert [experts_per_rank]
    int64); output row p of the expert-major layout reads input row
    permuted_indices[p] (expert_parallel.py:26-67). `total`, the number of
    received rows, defaults to the sum of the counts (one host sync, as the
    reference's torch.arange(total))."""
    require_gpu(tokens_per_expert_group)
    counts = tokens_per_expert_group.to(torch.int64).contiguous()
    if counts.numel() != experts_per_rank * num_ranks:
        raise ValueError(f"expected {num_ranks} x {experts_per_rank} counts, got {counts.numel()}")
    if total is None:
        total = int(counts.sum().item())
    idx = torch.empty(total, dtype=torch.int64, device=counts.device)
    ntok = torch.empty(experts_per_rank, dtype=torch.int64, device=counts.device)
    call("moe_ep_permute_indices", ptr(counts), experts_per_rank, num_ranks, total, ptr(idx), ptr(ntok),
         stream_of(counts))
    return idx, ntok


def _permute(x: torch.Tensor, num_tokens_per_expert: torch.Tensor, ep_degree: int, num_local_experts: int):
    """(input shape, x[permuted_indices], permuted_indices, per-expert counts);
    expert_parallel.py:70-74."""
    permuted_indices, num_tokens_per_expert = _generate_permute_indices(
        num_tokens_per_expert, num_local_experts, ep_degree
    )
    return x.shape, ops.gather_rows(x, permuted_indices), permuted_indices, num_tokens_per_expert


def _unpermute(out: torch.Tensor, input_shape, permuted_indices: torch.Tensor) -> torch.Tensor:
    """out_unpermuted[permuted_indices] = out; expert_parallel.py:77-80."""
    return ops.scatter_rows(out, permuted_indices, int(input_shape[0]))
