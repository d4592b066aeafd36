"""Auxiliary-loss-free load balancing: the optimizer step pre-hook that moves
each MoE layer's expert_bias toward balanced loads.

Mirrors register_moe_load_balancing_hook of
torchtitan/components/optimizer.py:337-444. The per-layer update
(``expert_bias += d - mean(d)``, ``d = coeff * sign(mean(t) - t)``,
``tokens_per_expert = 0``) runs as one HIP launch for every layer
(``moe_expert_bias_update``). When a process group is given, each rank first
floors its double-counted tokens (activation checkpointing) and the counts are
then summed across the group, in the reference's order.
"""

from __future__ import annotations

import ctypes

import torch
from torch import nn

from ._lib import call, require_gpu, stream_of
from .moe import MoE


def _is_recomputation_enabled(module: nn.Module) -> bool:
    """A block wrapped for non-reentrant activation checkpointing counts its
    tokens twice (optimizer.py:367-368, 389-394)."""
    try:
        from torch.distributed.algorithms._checkpoint.checkpoint_wrapper import CheckpointImpl
    except ImportError:  # pragma: no cover
        return False
    return getattr(module, "checkpoint_impl", None) is CheckpointImpl.NO_REENTRANT


def _moe_blocks(model_parts: list[nn.Module]) -> list[tuple[nn.Module, MoE]]:
    """(block, moe) for every MoE block: the reference's layers -> block.moe
    walk (optimizer.py:378-384), or every MoE module of a model without a
    ``layers`` dict."""
    found = []
    for part in model_parts:
        layers = getattr(part, "layers", None)
        if isinstance(layers, nn.ModuleDict):
            for block in layers.values():
                if getattr(block, "moe_enabled", False):
                    found.append((block, block.moe))
        else:
            found.extend((m, m) for m in part.modules() if isinstance(m, MoE))
    return found


def update_expert_bias(model_parts: list[nn.Module], group=None) -> None:
    """_update_expert_bias (optimizer.py:366-431) for every MoE layer of model_parts."""
    blocks = _moe_blocks(model_parts)
    if not blocks:
        return
    if any(moe.load_balance_coeff is None for _, moe in blocks):
        return  # the reference returns when a layer has no coefficient
    tpe = [moe.tokens_per_expert for _, moe in blocks]
    bias = [moe.expert_bias for _, moe in blocks]
    n_exp = tpe[0].numel()
    for t, b in zip(tpe, bias):
        if t.numel() != n_exp or b.numel() != n_exp or t.dtype != torch.float32 or b.dtype != torch.float32:
            raise ValueError("every MoE layer needs fp32 tokens_per_expert and expert_bias of one size")
        if not (t.is_contiguous() and b.is_contiguous()):
            raise ValueError("tokens_per_expert and expert_bias must be contiguous")
    halve = [_is_recomputation_enabled(block) for block, _ in blocks]
    if group is not None:
        # floor each rank's double-counted tokens before the sum, as the
        # reference does (optimizer.py:389-394 before :400-414)
        stacked = torch.stack([t // 2 if h else t for t, h in zip(tpe, halve)])
        torch.distributed.all_reduce(stacked, op=torch.distributed.ReduceOp.SUM, group=group)
        for t, row in zip(tpe, stacked):
            t.copy_(row)
        halve = [False] * len(halve)
    bias_update(tpe, bias, [float(moe.load_balance_coeff) for _, moe in blocks], halve)


def bias_update(tokens_per_expert: list[torch.Tensor], expert_bias: list[torch.Tensor], coeffs: list[float],
                halve: list[bool]) -> None:
    """One ``moe_expert_bias_update`` launch over the given layers' buffers ([E] fp32,
    contiguous, on one GPU): expert_bias += d - mean(d), d = coeff * sign(mean(t) - t),
    t = tokens_per_expert (// 2 where halve); tokens_per_expert = 0."""
    n = len(tokens_per_expert)
    if n == 0:
        return
    require_gpu(*tokens_per_expert, *expert_bias)
    ptrs = (ctypes.c_void_p * n)(*[t.data_ptr() for t in tokens_per_expert])
    bptrs = (ctypes.c_void_p * n)(*[b.data_ptr() for b in expert_bias])
    coeff = (ctypes.c_float * n)(*[float(c) for c in coeffs])
    hv = (ctypes.c_int32 * n)(*[int(bool(h)) for h in halve])
    call("moe_expert_bias_update", ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(bptrs, ctypes.c_void_p),
         ctypes.cast(coeff, ctypes.c_void_p), ctypes.cast(hv, ctypes.c_void_p), n, tokens_per_expert[0].numel(),
         stream_of(tokens_per_expert[0]))


def register_moe_load_balancing_hook(optimizers, model_parts: list[nn.Module], parallel_dims=None) -> None:
    """Registers the bias update as an optimizer step pre-hook when the MoE layers
    have a load_balance_coeff (optimizer.py:337-444). `optimizers` is anything
    with register_step_pre_hook (a torch optimizer or torchtitan's container)."""
    blocks = _moe_blocks(model_parts)
    if not blocks or not blocks[0][1].load_balance_coeff:
        return
    group = None
    if parallel_dims is not None and hasattr(parallel_dims, "get_optional_mesh"):
        mesh = parallel_dims.get_optional_mesh("loss")
        group = mesh.get_group() if mesh is not None else None
    optimizers.register_step_pre_hook(lambda *args, **kwargs: update_expert_bias(model_parts, group=group))
