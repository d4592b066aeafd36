"""HF <-> grouped-expert state-dict conversion (models/utils.py:19-387 offline
path, deepseek_v3 / gpt_oss key templates) on the CPU: key names follow the
reference's templates, expert e of a grouped weight is HF expert e, round
trips are exact, experts arriving out of order or interleaved across layers
stack in expert order, and the shard index math partitions the experts."""

import pytest
import torch

from torchtitan_amd.state_dict_adapter import (
    DEEPSEEK_V3_MOE_FROM_HF,
    GPT_OSS_MOE_FROM_HF,
    MoEStateDictAdapter,
    shard_indices,
    strided_shard_indices,
)


def _moe_state(layers=(0, 3), e=4, d=8, h=6, hs=5):
    g = torch.Generator().manual_seed(0)
    sd = {}
    for L in layers:
        p = f"layers.{L}.moe."
        sd[p + "experts.w1"] = torch.randn(e, h, d, generator=g)
        sd[p + "experts.w3"] = torch.randn(e, h, d, generator=g)
        sd[p + "experts.w2"] = torch.randn(e, d, h, generator=g)
        sd[p + "router.gate.weight"] = torch.randn(e, d, generator=g)
        sd[p + "expert_bias"] = torch.randn(e, generator=g)
        sd[p + "shared_experts.w1.weight"] = torch.randn(hs, d, generator=g)
        sd[p + "shared_experts.w3.weight"] = torch.randn(hs, d, generator=g)
        sd[p + "shared_experts.w2.weight"] = torch.randn(d, hs, generator=g)
    return sd


def test_to_hf_names_and_splits_experts():
    sd = _moe_state()
    hf = MoEStateDictAdapter(DEEPSEEK_V3_MOE_FROM_HF, num_experts=4).to_hf(sd)
    assert len(hf) == 2 * (3 * 4 + 5)
    assert torch.equal(hf["model.layers.3.mlp.experts.2.gate_proj.weight"], sd["layers.3.moe.experts.w1"][2])
    assert torch.equal(hf["model.layers.0.mlp.experts.1.up_proj.weight"], sd["layers.0.moe.experts.w3"][1])
    assert torch.equal(hf["model.layers.0.mlp.experts.3.down_proj.weight"], sd["layers.0.moe.experts.w2"][3])
    assert hf["model.layers.0.mlp.experts.3.down_proj.weight"].shape == (8, 6)
    assert torch.equal(hf["model.layers.3.mlp.gate.e_score_correction_bias"], sd["layers.3.moe.expert_bias"])
    assert torch.equal(hf["model.layers.0.mlp.shared_experts.down_proj.weight"],
                       sd["layers.0.moe.shared_experts.w2.weight"])


def test_round_trip_and_out_of_order_experts():
    sd = _moe_state()
    ad = MoEStateDictAdapter(DEEPSEEK_V3_MOE_FROM_HF, num_experts=4)
    hf = ad.to_hf(sd)
    items = list(hf.items())
    g = torch.Generator().manual_seed(1)
    shuffled = dict(items[i] for i in torch.randperm(len(items), generator=g).tolist())
    back = ad.from_hf(shuffled)
    assert set(back) == set(sd)
    for k in sd:
        assert torch.equal(back[k], sd[k]), k


def test_incomplete_experts_are_not_stacked_and_unknown_keys():
    ad = MoEStateDictAdapter(DEEPSEEK_V3_MOE_FROM_HF, num_experts=4)
    hf = {f"model.layers.1.mlp.experts.{e}.gate_proj.weight": torch.full((2, 3), float(e)) for e in (0, 2, 3)}
    assert ad.from_hf(hf) == {}
    hf["model.layers.1.mlp.experts.1.gate_proj.weight"] = torch.full((2, 3), 1.0)
    w1 = ad.from_hf(hf)["layers.1.moe.experts.w1"]
    assert w1[:, 0, 0].tolist() == [0.0, 1.0, 2.0, 3.0]
    with pytest.raises(KeyError):
        ad.from_hf({"model.layers.1.self_attn.o_proj.weight": torch.zeros(1)})
    with pytest.raises(KeyError):
        ad.to_hf({"layers.1.attention.wo.weight": torch.zeros(1)})
    lax = MoEStateDictAdapter(DEEPSEEK_V3_MOE_FROM_HF, num_experts=4, strict=False)
    assert lax.to_hf({"layers.1.attention.wo.weight": torch.zeros(1)}) == {}


def test_gpt_oss_keys_are_renamed_without_reshaping():
    ad = MoEStateDictAdapter(GPT_OSS_MOE_FROM_HF, num_experts=4)
    w = torch.randn(4, 12, 8)
    hf = ad.to_hf({"layers.2.moe.experts.mlp1_weight": w, "layers.2.moe.experts.mlp2_bias": torch.zeros(4, 8)})
    assert set(hf) == {"model.layers.2.mlp.experts.gate_up_proj_blocks", "model.layers.2.mlp.experts.down_proj_bias"}
    assert hf["model.layers.2.mlp.experts.gate_up_proj_blocks"] is w
    assert ad.from_hf(hf)["layers.2.moe.experts.mlp1_weight"] is w


def test_shard_index_math_partitions_the_experts():
    # the reference's docstring grid: StridedShard degree 3 x Shard degree 2 over 12 experts
    assert strided_shard_indices(3, 1, 2, 0, 12) == (2, 4)
    assert strided_shard_indices(3, 0, 2, 1, 12) == (6, 8)
    for sd_deg, s_deg, n in ((3, 2, 12), (2, 4, 64), (1, 8, 256)):
        covered = sorted(strided_shard_indices(sd_deg, a, s_deg, b, n) for a in range(sd_deg) for b in range(s_deg))
        assert covered[0][0] == 0 and covered[-1][1] == n
        assert all(covered[i][1] == covered[i + 1][0] for i in range(len(covered) - 1))
    assert shard_indices(256, 8, 3) == (96, 128)
    with pytest.raises(ValueError):
        shard_indices(10, 4, 0)
    with pytest.raises(ValueError):
        strided_shard_indices(3, 0, 2, 0, 10)
