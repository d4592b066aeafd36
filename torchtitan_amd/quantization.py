"""fp8 and MXFP8 for the MoE experts, with the interface of the reference's converters.

Mirrors ``Float8GroupedMMConverter`` (torchtitan/components/quantization/float8.py:220-300),
``MXFP8Converter`` (quantization/mx.py:25-134) and ``PAD_MULTIPLE_MAP`` /
``find_pad_multiple`` (quantization/__init__.py:34-57):
``<Converter>.Config(fqns=[...]).build(...).convert(model)`` switches every
``GroupedExperts`` whose fully qualified name contains one of ``fqns`` to the
MI355X quantized grouped GEMMs: fp8 e4m3 with dynamic rowwise scales, or
MXFP8 (e4m3 elements, one e8m0 scale per 32 along the contraction, RCEIL);
fp32 accumulation, bf16 outputs. Parameters stay bf16/fp32 master weights and
the state_dict is unchanged; quantization happens inside each forward and
backward.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, field

import torch
from torch import nn

from .configurable import Configurable
from .moe import GroupedExperts

__all__ = ["Float8GroupedMMConverter", "MXFP8Converter", "PAD_MULTIPLE_MAP", "find_pad_multiple"]

logger = logging.getLogger(__name__)


def has_gfx950() -> bool:
    """True when the current GPU is an MI355X-class CDNA4 part (gfx950), whose
    fp8 e4m3 and block-scaled MFMAs these kernels use. The reference's converters
    check for CUDA SM89 / SM100 instead (torchtitan/tools/utils.py:20-33)."""
    if not torch.cuda.is_available():
        return False
    arch = getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", "")
    return arch.split(":")[0] == "gfx950"

# token-group alignment of quantized grouped GEMMs (fp8: 16 one-byte elements;
# MXFP8: one 32-element scaling block)
PAD_MULTIPLE_MAP: dict[str, int] = {"float8": 16, "mxfp8": 32}


class Float8GroupedMMConverter(Configurable):
    @dataclass(kw_only=True, slots=True)
    class Config(Configurable.Config):
        fqns: list[str] | str = field(default_factory=list)

    def __init__(self, config: Config, *, parallel_dims, model_compile_enabled: bool):
        """Checks as float8.py:238-256 does: the hardware first, then the MoE
        training prototype's limits (no pipeline or context parallelism)."""
        self.fqns = _split_fqns(config.fqns)
        if not has_gfx950():
            raise ValueError("Float8 MoE training only supported on gfx950 (MI355X).")
        if not model_compile_enabled:
            logger.info("float8 MoE: the grouped GEMMs are hand-written kernels; compile is not needed for speed")
        assert not parallel_dims.pp_enabled, (
            "Float8 MoE training prototype does not yet support pipeline parallelism"
        )
        assert not parallel_dims.cp_enabled, (
            "Float8 MoE training prototype does not yet support context parallelism"
        )
        self.enabled = True

    def convert(self, model: nn.Module) -> list[str]:
        """Switches the matching GroupedExperts to fp8; returns their names."""
        return _mark_experts(model, self.fqns, "float8")

    def post_optimizer_hook(self, model) -> None:
        pass


def _split_fqns(fqns: list[str] | str) -> list[str]:
    return [f for f in fqns.split(",") if f] if isinstance(fqns, str) else list(fqns)


def _mark_experts(model: nn.Module, fqns: list[str], attr: str) -> list[str]:
    converted = []
    for name, mod in model.named_modules():
        if isinstance(mod, GroupedExperts) and any(f in name for f in fqns):
            setattr(mod, attr, True)
            converted.append(name)
    return converted


class MXFP8Converter(Configurable):
    """MXFP8 grouped GEMMs for the matching experts (torchao's
    MXFP8TrainingOpConfig.from_recipe(MXFP8TrainingRecipe(recipe_name)) in the
    reference, mx.py:85-128). The kernels take ragged token groups, so no
    padding of the routed rows is needed without expert parallelism either."""

    RECIPES = ("mxfp8_rceil",)

    @dataclass(kw_only=True, slots=True)
    class Config(Configurable.Config):
        recipe_name: str = "mxfp8_rceil"
        fqns: list[str] | str = field(default_factory=list)

    def __init__(self, config: Config, *, parallel_dims, model_compile_enabled: bool):
        """Checks as mx.py:51-80 does: the hardware (block-scaled MFMA, gfx950
        here, SM100 there), then the recipe. Ragged token groups need no
        padding in these kernels, with or without expert parallelism."""
        self.enabled = False
        assert has_gfx950(), "MXFP8 is only supported on gfx950 (MI355X)"
        if config.recipe_name not in self.RECIPES:
            raise ValueError(f"unknown MXFP8 recipe {config.recipe_name!r}; options: {list(self.RECIPES)}")
        if not model_compile_enabled:
            logger.info("MXFP8 MoE: the grouped GEMMs are hand-written kernels; compile is not needed for speed")
        self.recipe_name = config.recipe_name
        self.fqns = _split_fqns(config.fqns)
        self.pad_token_groups_for_grouped_mm = not parallel_dims.ep_enabled
        self.config = config
        self.enabled = True

    def convert(self, model: nn.Module) -> list[str]:
        """Switches the matching GroupedExperts to MXFP8; returns their names."""
        if not self.enabled:
            return []
        return _mark_experts(model, self.fqns, "mxfp8")

    def post_optimizer_hook(self, model) -> None:
        pass


def find_pad_multiple(converters: list) -> int | None:
    """Token-group pad multiple needed by the configured quantized grouped GEMMs."""
    for c in converters:
        if isinstance(c, Float8GroupedMMConverter.Config):
            return PAD_MULTIPLE_MAP["float8"]
        if isinstance(c, MXFP8Converter.Config):
            return PAD_MULTIPLE_MAP["mxfp8"]
    return None
