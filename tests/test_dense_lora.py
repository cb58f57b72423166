"""Host-side construction and validation of the dense LoRA linears (no GPU
calls: the weights stay on the CPU and nothing is launched)."""
import pytest
import torch

from art_amd.megatron.dense_lora import (DenseLoRALinear, Placement, SelfAttentionLinearProjLoRA,
                                         SelfAttentionLinearQKVLoRA, SharedExpertsLinearFC1LoRA,
                                         SharedExpertsLinearFC2LoRA)
from art_amd.megatron.lora import LoRA


def _w(out, inp):
    return torch.zeros(out, inp, dtype=torch.bfloat16)


def _cols(pl: Placement):
    return [g * pl.period + pl.offset + j for g in range(pl.groups) for j in range(pl.width)]


def test_placements_tile_the_output():
    fc1 = SharedExpertsLinearFC1LoRA("m.shared_expert", _w(640, 256), 8, 16)
    (_, gate), (_, up) = fc1.linear.segments
    assert _cols(gate) == list(range(320)) and _cols(up) == list(range(320, 640))
    assert fc1.gate_lora.adapter_model_prefix == "m.shared_expert.gate_proj"
    assert fc1.up_lora.B_T.shape == (8, 320)
    fc2 = SharedExpertsLinearFC2LoRA("m.shared_expert", _w(256, 320), 8, 16)
    assert fc2.row_parallel_lora.lora.adapter_model_prefix == "m.shared_expert.down_proj"
    proj = SelfAttentionLinearProjLoRA("a.o_proj", _w(96, 128), 4, 8)
    assert _cols(proj.linear.segments[0][1]) == list(range(96))


@pytest.mark.parametrize("gate", [False, True])
def test_qkv_placement_matches_grouped_query_layout(gate):
    heads, groups, d = 6, 3, 16
    hpg = heads // groups
    qw = hpg * d * (2 if gate else 1)
    qkv = SelfAttentionLinearQKVLoRA("l.self_attn", _w(groups * (qw + 2 * d), 64), 4, 8,
                                     num_attention_heads=heads, num_query_groups=groups,
                                     kv_channels=d, attention_output_gate=gate)
    (_, q), (_, k), (_, v) = qkv.linear.segments
    cols = _cols(q) + _cols(k) + _cols(v)
    assert sorted(cols) == list(range(groups * (qw + 2 * d)))       # disjoint cover
    # group g's k slot starts right after its q (and gate) heads
    assert _cols(k)[:d] == list(range(qw, qw + d)) and _cols(v)[d] == (qw + 2 * d) + qw + d
    assert qkv.q_proj_lora.B_T.shape == (4, groups * qw)
    assert qkv.k_proj_lora.adapter_model_prefix == "l.self_attn.k_proj"
    assert qkv.q_and_gate_out_features_per_rank == groups * qw
    assert qkv.kv_out_features_per_rank == groups * d


def test_qkv_targets_and_shape_errors():
    qkv = SelfAttentionLinearQKVLoRA("l", _w(2 * (32 + 32), 64), 4, 8, num_attention_heads=4,
                                     num_query_groups=2, kv_channels=16,
                                     target_modules={"q_proj"})
    assert qkv.k_proj_lora is None and qkv.v_proj_lora is None and len(qkv.linear.segments) == 1
    with pytest.raises(ValueError, match="divisible"):
        SelfAttentionLinearQKVLoRA("l", _w(192, 64), 4, 8, num_attention_heads=5,
                                   num_query_groups=2, kv_channels=16)
    with pytest.raises(ValueError, match="packing needs"):
        SelfAttentionLinearQKVLoRA("l", _w(190, 64), 4, 8, num_attention_heads=4,
                                   num_query_groups=2, kv_channels=16)
    with pytest.raises(ValueError, match="even"):
        SharedExpertsLinearFC1LoRA("m", _w(63, 64), 4, 8)


def test_dense_linear_rejects_bad_segments():
    w = _w(64, 32)
    lora = LoRA("p", 32, 64, 4, 8, torch.bfloat16, "cpu")
    with pytest.raises(ValueError, match="does not tile"):
        DenseLoRALinear(w, [(lora, Placement(1, 32, 0, 64))])
    with pytest.raises(ValueError, match="do not fit"):
        DenseLoRALinear(w, [(lora, Placement.columns(0, 32, 64))])
    experts = LoRA("p.{expert}", 32, 64, 4, 8, torch.bfloat16, "cpu", num_local_experts=2)
    with pytest.raises(ValueError, match="one expert"):
        DenseLoRALinear(w, [(experts, Placement.columns(0, 64, 64))])
