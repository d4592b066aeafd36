"""HF <-> grouped-expert state-dict conversion for the MoE layer.

Mirrors ``MoEStateDictAdapter`` (torchtitan/models/utils.py:19-387) on one
device: HF checkpoints keep one 2-D weight per expert
(``model.layers.{L}.mlp.experts.{e}.gate_proj.weight``, ``[H, D]``), the
layer here keeps a 3-D parameter per projection (``layers.{L}.moe.experts.w1``,
``[E, H, D]``). ``to_hf`` splits (views, no copy), ``from_hf`` collects the
experts of a layer and stacks them once all ``num_experts`` have arrived
(``_concatenate_expert_weights``, utils.py:346-386); every other key is
renamed through the same template map (deepseek_v3/state_dict_adapter.py:
98-218). The expert-dimension index math of the sharded (DTensor) path
(utils.py:44-159) is kept as pure functions; building DTensors needs a device
mesh and is not part of this one-GPU layer.
"""

from __future__ import annotations

import re
from typing import Any

import torch

__all__ = [
    "DEEPSEEK_V3_MOE_FROM_HF",
    "GPT_OSS_MOE_FROM_HF",
    "MoEStateDictAdapter",
    "shard_indices",
    "strided_shard_indices",
]

# The MoE entries of the reference's HF -> torchtitan key templates
# (deepseek_v3/state_dict_adapter.py:46-54; gpt_oss/state_dict_adapter.py:35-41).
DEEPSEEK_V3_MOE_FROM_HF: dict[str, str] = {
    "model.layers.{}.mlp.experts.{}.gate_proj.weight": "layers.{}.moe.experts.w1",
    "model.layers.{}.mlp.experts.{}.up_proj.weight": "layers.{}.moe.experts.w3",
    "model.layers.{}.mlp.experts.{}.down_proj.weight": "layers.{}.moe.experts.w2",
    "model.layers.{}.mlp.gate.weight": "layers.{}.moe.router.gate.weight",
    "model.layers.{}.mlp.shared_experts.gate_proj.weight": "layers.{}.moe.shared_experts.w1.weight",
    "model.layers.{}.mlp.shared_experts.up_proj.weight": "layers.{}.moe.shared_experts.w3.weight",
    "model.layers.{}.mlp.shared_experts.down_proj.weight": "layers.{}.moe.shared_experts.w2.weight",
    "model.layers.{}.mlp.gate.e_score_correction_bias": "layers.{}.moe.expert_bias",
}

GPT_OSS_MOE_FROM_HF: dict[str, str] = {
    "model.layers.{}.mlp.experts.gate_up_proj_blocks": "layers.{}.moe.experts.mlp1_weight",
    "model.layers.{}.mlp.experts.gate_up_proj_bias": "layers.{}.moe.experts.mlp1_bias",
    "model.layers.{}.mlp.experts.down_proj_blocks": "layers.{}.moe.experts.mlp2_weight",
    "model.layers.{}.mlp.experts.down_proj_bias": "layers.{}.moe.experts.mlp2_bias",
    "model.layers.{}.mlp.router.weight": "layers.{}.moe.router.gate.weight",
    "model.layers.{}.mlp.router.bias": "layers.{}.moe.router.gate.bias",
}


def shard_indices(dim_size: int, degree: int, rank: int) -> tuple[int, int]:
    """[start, end) of `rank`'s block under one Shard(dim) placement (utils.py:140-150)."""
    block = dim_size // degree
    if block * degree != dim_size:
        raise ValueError(f"dim size {dim_size} cannot be evenly divided by shard degree {degree}")
    return block * rank, block * rank + block


def strided_shard_indices(strided_degree: int, strided_rank: int, shard_degree: int, shard_rank: int,
                          dim_size: int) -> tuple[int, int]:
    """[start, end) under [StridedShard(dim), Shard(dim)] (utils.py:44-95): the
    inner Shard rank picks a group of strided_degree blocks, the strided rank
    the block inside it."""
    block = dim_size // (strided_degree * shard_degree)
    if block * strided_degree * shard_degree != dim_size:
        raise ValueError(f"Not supported split for strided_shard_dim_degree {strided_degree}, "
                         f"shard_dim_degree {shard_degree}, dim_size_to_split {dim_size}")
    start = block * (strided_degree * shard_rank + strided_rank)
    return start, start + block


class MoEStateDictAdapter:
    """Offline HF <-> torchtitan conversion of MoE-layer state dicts.

    ``from_hf_map`` maps HF key templates to torchtitan ones; a template with
    two ``{}`` on the HF side (layer, expert) is a per-expert weight that maps
    to one grouped 3-D parameter. Keys without a template raise ``KeyError``
    (as deepseek_v3/state_dict_adapter.py:98-157) or, with ``strict=False``,
    are dropped (as gpt_oss/state_dict_adapter.py:67-97)."""

    def __init__(self, from_hf_map: dict[str, str], num_experts: int, strict: bool = True):
        self.from_hf_map = dict(from_hf_map)
        self.to_hf_map = {v: k for k, v in self.from_hf_map.items()}
        self.num_experts = num_experts
        self.strict = strict

    @staticmethod
    def _split_experts_weights(weight: torch.Tensor, n_experts: int) -> tuple[torch.Tensor, ...]:
        return torch.split(weight, weight.shape[0] // n_experts, dim=0)

    @staticmethod
    def _concatenate_expert_weights(expert_weights_by_layer: dict, abstract_key: str, layer_num: str,
                                    n_experts: int) -> torch.Tensor | None:
        experts = expert_weights_by_layer[layer_num][abstract_key]
        if len(experts) < n_experts:
            return None
        stacked = torch.stack([experts[i] for i in sorted(experts)], dim=0)
        del expert_weights_by_layer[layer_num][abstract_key]
        if not expert_weights_by_layer[layer_num]:
            del expert_weights_by_layer[layer_num]
        return stacked

    def _is_per_expert(self, hf_template: str) -> bool:
        return hf_template.count("{}") == 2

    def to_hf(self, state_dict: dict[str, Any]) -> dict[str, Any]:
        hf: dict[str, Any] = {}
        for key, value in state_dict.items():
            abstract = re.sub(r"(\d+)", "{}", key, count=1)
            if abstract not in self.to_hf_map:
                if key in self.to_hf_map:
                    hf[self.to_hf_map[key]] = value
                elif self.strict:
                    raise KeyError(f"no HF key for {key!r}")
                continue
            layer = re.search(r"\d+", key).group(0)
            hf_template = self.to_hf_map[abstract]
            if self._is_per_expert(hf_template):
                for e, w in enumerate(self._split_experts_weights(value, self.num_experts)):
                    hf[hf_template.format(layer, e)] = w.squeeze()
            else:
                hf[hf_template.format(layer)] = value
        return hf

    def from_hf(self, hf_state_dict: dict[str, Any]) -> dict[str, Any]:
        out: dict[str, Any] = {}
        pending: dict[str, dict[str, dict[int, torch.Tensor]]] = {}
        for key, value in hf_state_dict.items():
            two = re.sub(r"(\d+)", "{}", key, count=2)
            if two in self.from_hf_map and self._is_per_expert(two):
                layer, expert = re.findall(r"\d+", key)[:2]
                tt_template = self.from_hf_map[two]
                pending.setdefault(layer, {}).setdefault(tt_template, {})[int(expert)] = value
                stacked = self._concatenate_expert_weights(pending, tt_template, layer, self.num_experts)
                if stacked is not None:
                    out[tt_template.format(layer)] = stacked
                continue
            one = re.sub(r"(\d+)", "{}", key, count=1)
            if one in self.from_hf_map:
                out[self.from_hf_map[one].format(re.search(r"\d+", key).group(0))] = value
            elif key in self.from_hf_map:
                out[self.from_hf_map[key]] = value
            elif self.strict:
                raise KeyError(f"no torchtitan key for HF key {key!r}")
        return out
