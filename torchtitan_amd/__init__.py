"""MI355X-native MoE layer hot path, drop-in for torchtitan's MoE building blocks.

Public surface (mirrors torchtitan/models/common/{moe,feed_forward,linear}.py):
``MoE``, ``TokenChoiceTopKRouter``, ``TokenReorderer``, ``GroupedExperts``,
``FeedForward``, ``Linear`` and the module-level ``_run_experts_grouped_mm`` /
``_run_experts_for_loop`` swap points. The arithmetic runs in
``libmoe_mi355x.so`` (HIP kernels for gfx950, C ABI in include/moe_mi355x.h)
through the ``moe_mi355x::*`` torch custom ops in ``torchtitan_amd.ops``.
"""

from .configurable import Configurable, Module
from .feed_forward import FeedForward, compute_ffn_hidden_dim
from .linear import Linear
from .moe import (
    GroupedExperts,
    MoE,
    ReorderResult,
    TokenChoiceTopKRouter,
    TokenReorderer,
    _run_experts_for_loop,
    _run_experts_grouped_mm,
)

__all__ = [
    "Configurable",
    "FeedForward",
    "GroupedExperts",
    "Linear",
    "MoE",
    "Module",
    "ReorderResult",
    "TokenChoiceTopKRouter",
    "TokenReorderer",
    "compute_ffn_hidden_dim",
    "_run_experts_for_loop",
    "_run_experts_grouped_mm",
]
