"""fp8 for the MoE experts, with the interface of the reference's converter.

Mirrors ``Float8GroupedMMConverter`` (torchtitan/components/quantization/float8.py:220-300)
and ``PAD_MULTIPLE_MAP`` / ``find_pad_multiple`` (quantization/__init__.py:34-57):
``Float8GroupedMMConverter.Config(fqns=[...]).build(...).convert(model)`` switches
every ``GroupedExperts`` whose fully qualified name contains one of ``fqns`` to
the MI355X fp8 e4m3 grouped GEMMs (dynamic rowwise scaling, fp32 accumulation,
bf16 outputs). Parameters stay bf16/fp32 master weights and the state_dict is
unchanged; quantization happens inside each forward and backward.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from torch import nn

from .configurable import Configurable
from .moe import GroupedExperts

__all__ = ["Float8GroupedMMConverter", "PAD_MULTIPLE_MAP", "find_pad_multiple"]

# token-group alignment of quantized grouped GEMMs (fp8: 16 one-byte elements)
PAD_MULTIPLE_MAP: dict[str, int] = {"float8": 16, "mxfp8": 32}


class Float8GroupedMMConverter(Configurable):
    @dataclass(kw_only=True, slots=True)
    class Config(Configurable.Config):
        fqns: list[str] | str = field(default_factory=list)

    def __init__(self, config: Config, **_unused):
        fqns = config.fqns
        self.fqns = [f for f in fqns.split(",") if f] if isinstance(fqns, str) else list(fqns)
        self.enabled = True

    def convert(self, model: nn.Module) -> list[str]:
        """Switches the matching GroupedExperts to fp8; returns their names."""
        converted = []
        for name, mod in model.named_modules():
            if isinstance(mod, GroupedExperts) and any(f in name for f in self.fqns):
                mod.float8 = True
                converted.append(name)
        return converted

    def post_optimizer_hook(self, model) -> None:
        pass


def find_pad_multiple(converters: list) -> int | None:
    """Token-group pad multiple needed by the configured quantized grouped GEMMs."""
    for c in converters:
        if isinstance(c, Float8GroupedMMConverter.Config):
            return PAD_MULTIPLE_MAP["float8"]
    return None
