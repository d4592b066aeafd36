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

from dataclasses import dataclass, field

from torch import nn

from .configurable import Configurable
from .moe import GroupedExperts

__all__ = ["Float8GroupedMMConverter", "MXFP8Converter", "PAD_MULTIPLE_MAP", "find_pad_multiple"]

# token-group alignment of quantized grouped GEMMs (fp8: 16 one-byte elements;
# MXFP8: one 32-element scaling block)
PAD_MULTIPLE_MAP: dict[str, int] = {"float8": 16, "mxfp8": 32}


class Float8GroupedMMConverter(Configurable):
    @dataclass(kw_only=True, slots=True)
    class Config(Configurable.Config):
        fqns: list[str] | str = field(default_factory=list)

    def __init__(self, config: Config, **_unused):
        self.fqns = _split_fqns(config.fqns)
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

    def __init__(self, config: Config, **_unused):
        if config.recipe_name not in self.RECIPES:
            raise ValueError(f"unknown MXFP8 recipe {config.recipe_name!r}; options: {list(self.RECIPES)}")
        self.recipe_name = config.recipe_name
        self.fqns = _split_fqns(config.fqns)
        self.enabled = True

    def convert(self, model: nn.Module) -> list[str]:
        """Switches the matching GroupedExperts to MXFP8; returns their names."""
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
