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


def _permute_and_pad(x: torch.Tensor, num_tokens_per_expert_group: torch.Tensor, ep_degree: int,
                     num_local_experts: int, pad_multiple: int):
    """The permute of TorchAOExpertParallel._token_dispatch (expert_parallel.py:537-551,
    torchao's permute_and_pad): expert-major rows with every expert's group padded by
    zero rows to a multiple of pad_multiple (16 fp8, 32 MXFP8). Returns
    (input_shape with one extra row, padded routed input, permuted_indices (padding
    rows index that extra zero row), padded per-expert counts, int32 group end offsets)."""
    require_gpu(x, num_tokens_per_expert_group)
    counts = num_tokens_per_expert_group.to(torch.int64).contiguous()
    if counts.numel() != ep_degree * num_local_experts:
        raise ValueError(f"expected {ep_degree} x {num_local_experts} counts, got {counts.numel()}")
    per_expert = counts.view(ep_degree, num_local_experts).sum(0)
    total_padded = int(((per_expert + pad_multiple - 1) // pad_multiple * pad_multiple).sum().item())
    idx = torch.empty(total_padded, dtype=torch.int64, device=x.device)
    padded = torch.empty(num_local_experts, dtype=torch.int64, device=x.device)
    offsets = torch.empty(num_local_experts, dtype=torch.int32, device=x.device)
    call("moe_ep_permute_pad_indices", ptr(counts), num_local_experts, ep_degree, pad_multiple, total_padded,
         ptr(idx), ptr(padded), ptr(offsets), stream_of(counts))
    input_shape = torch.Size((x.shape[0] + 1, *x.shape[1:]))
    return input_shape, ops.gather_rows(x, idx), idx, padded, offsets


def _unpermute_padded(out: torch.Tensor, input_shape, permuted_indices: torch.Tensor) -> torch.Tensor:
    """TorchAOExpertParallel._token_combine's unpermute (expert_parallel.py:556-562):
    rows back to rank-major order, the padding rows (which target the extra last row
    of input_shape) dropped."""
    return ops.scatter_rows(out, permuted_indices, int(input_shape[0]) - 1)
