"""Adapter layout conversions of the grouped-MoE layer (host logic, CPU).

Golden behaviour from the reference's own tests: the arange fixtures of
tests/integration/megatron/lora/test_lora_disk_codecs.py:474-530 (fused Qwen3
MoE block -> per-expert tensors), :533-592 (PEFT fused checkpoint -> vLLM
orientation, config rewrite), :595-635 (swapped PEFT block through both steps)
and :637-700 (target-parameter orientation).  The megatron-bridge pair export
and the fused export of ART's factors are pinned by the adapter they apply:
scale * B A must be the same linear map in every layout.
"""
import json

import pytest
import torch

from art_amd.megatron import adapter_io as A
from art_amd.megatron.lora import LoRA

PREFIX = "base_model.model.model.layers.0.mlp.experts"


def _fused_fixture(rank=2):
    """test_lora_disk_codecs.py:479-530: standard-orientation fused block and
    the per-expert tensors it expands to."""
    hidden, inter, e_n = 3, 4, 2
    gu_a = torch.arange(e_n * rank * hidden, dtype=torch.float32).reshape(e_n * rank, hidden)
    d_a = torch.arange(e_n * rank * inter, dtype=torch.float32).reshape(e_n * rank, inter) + 100
    gu_b = [torch.arange(2 * inter * rank, dtype=torch.float32).reshape(2 * inter, rank) + 200 + 100 * e
            for e in range(e_n)]
    d_b = [torch.arange(hidden * rank, dtype=torch.float32).reshape(hidden, rank) + 500 + 100 * e
           for e in range(e_n)]
    fused = {f"{PREFIX}.base_layer.lora_A.weight": gu_a,
             f"{PREFIX}.base_layer.lora_B.weight": A.pack_lora_b_by_expert(gu_b),
             f"{PREFIX}.lora_A.weight": d_a,
             f"{PREFIX}.lora_B.weight": A.pack_lora_b_by_expert(d_b)}
    expected = {}
    for e in range(e_n):
        rows = slice(e * rank, (e + 1) * rank)
        gate_b, up_b = gu_b[e].split(inter, dim=0)
        p = f"{PREFIX}.{e}"
        expected[f"{p}.gate_proj.lora_A.weight"] = gu_a[rows]
        expected[f"{p}.gate_proj.lora_B.weight"] = gate_b
        expected[f"{p}.up_proj.lora_A.weight"] = gu_a[rows]
        expected[f"{p}.up_proj.lora_B.weight"] = up_b
        expected[f"{p}.down_proj.lora_A.weight"] = d_a[rows]
        expected[f"{p}.down_proj.lora_B.weight"] = d_b[e]
    return fused, expected


def _assert_same(got, expected):
    assert set(got) == set(expected)
    for k in expected:
        assert torch.equal(got[k], expected[k]), k


def test_pack_lora_b_by_expert_layout_and_inverse():
    blocks = [torch.arange(6, dtype=torch.float32).reshape(3, 2) + 10 * e for e in range(4)]
    packed = A.pack_lora_b_by_expert(blocks)
    assert packed.shape == (3, 8)
    for e in range(4):      # column i * E + e holds expert e's rank column i
        for i in range(2):
            assert torch.equal(packed[:, i * 4 + e], blocks[e][:, i])
    back = A.packed_lora_b_by_expert(packed, num_experts=4, rank=2)
    assert all(torch.equal(back[e], blocks[e]) for e in range(4))


def test_fused_standard_orientation_expands_per_expert():
    fused, expected = _fused_fixture()
    out, cfg = A.to_vllm_lora_tensors(fused, adapter_config={"r": 2, "target_modules": ["q_proj"]})
    _assert_same(out, expected)
    assert cfg["target_modules"] == ["q_proj", "experts"]


def test_peft_fused_checkpoint_converts_to_vllm_orientation(tmp_path):
    """test_lora_disk_codecs.py:533-592."""
    safetensors = pytest.importorskip("safetensors.torch")
    t = {f"{PREFIX}.base_layer.lora_A.weight": torch.arange(16, dtype=torch.float32).reshape(2, 8),
         f"{PREFIX}.base_layer.lora_B.weight": torch.arange(6, dtype=torch.float32).reshape(3, 2) + 100,
         f"{PREFIX}.lora_A.weight": torch.arange(6, dtype=torch.float32).reshape(2, 3) + 200,
         f"{PREFIX}.lora_B.weight": torch.arange(8, dtype=torch.float32).reshape(4, 2) + 300}
    safetensors.save_file(t, str(tmp_path / "adapter_model.safetensors"))
    (tmp_path / "adapter_config.json").write_text(json.dumps({
        "r": 1, "lora_alpha": 1, "target_modules": ["q_proj"],
        "target_parameters": ["model.layers.0.mlp.experts.gate_up_proj",
                              "model.layers.0.mlp.experts.down_proj"]}))
    assert A.convert_checkpoint_if_needed(str(tmp_path))
    got = safetensors.load_file(str(tmp_path / "adapter_model.safetensors"))
    _assert_same(got, {
        f"{PREFIX}.base_layer.lora_A.weight": t[f"{PREFIX}.base_layer.lora_B.weight"].T.contiguous(),
        f"{PREFIX}.base_layer.lora_B.weight": t[f"{PREFIX}.base_layer.lora_A.weight"].T.contiguous(),
        f"{PREFIX}.lora_A.weight": t[f"{PREFIX}.lora_B.weight"].T.contiguous(),
        f"{PREFIX}.lora_B.weight": t[f"{PREFIX}.lora_A.weight"].T.contiguous()})
    cfg = json.loads((tmp_path / "adapter_config.json").read_text())
    assert cfg["target_modules"] == ["q_proj", "experts"] and "target_parameters" not in cfg
    assert not A.convert_checkpoint_if_needed(str(tmp_path))   # already converted: no-op


def test_swapped_peft_block_normalises_to_per_expert(tmp_path):
    """test_lora_disk_codecs.py:595-635: the fixture stored A/B-swapped (PEFT),
    converted, then expanded, gives the fixture's per-expert tensors."""
    safetensors = pytest.importorskip("safetensors.torch")
    fused, expected = _fused_fixture()
    swapped = {f"{PREFIX}.base_layer.lora_A.weight": fused[f"{PREFIX}.base_layer.lora_B.weight"].T.contiguous(),
               f"{PREFIX}.base_layer.lora_B.weight": fused[f"{PREFIX}.base_layer.lora_A.weight"].T.contiguous(),
               f"{PREFIX}.lora_A.weight": fused[f"{PREFIX}.lora_B.weight"].T.contiguous(),
               f"{PREFIX}.lora_B.weight": fused[f"{PREFIX}.lora_A.weight"].T.contiguous()}
    safetensors.save_file(swapped, str(tmp_path / "adapter_model.safetensors"))
    (tmp_path / "adapter_config.json").write_text(json.dumps({
        "r": 2, "lora_alpha": 4, "target_modules": ["q_proj"],
        "target_parameters": ["model.layers.0.mlp.experts.gate_up_proj"]}))
    A.convert_checkpoint_if_needed(str(tmp_path))
    out, cfg = A.to_vllm_lora_tensors(safetensors.load_file(str(tmp_path / "adapter_model.safetensors")),
                                      adapter_config={"r": 2, "target_modules": ["q_proj"]})
    _assert_same(out, expected)
    assert "experts" in cfg["target_modules"]


def test_target_parameter_orientation_expands_per_expert():
    """test_lora_disk_codecs.py:637-700 (expected tensors restated there)."""
    rank, hidden, inter, e_n = 2, 3, 4, 2
    gu_a = torch.arange(e_n * rank * 2 * inter, dtype=torch.float32).reshape(e_n * rank, 2 * inter)
    gu_b = torch.arange(hidden * e_n * rank, dtype=torch.float32).reshape(hidden, e_n * rank) + 100
    d_a = torch.arange(e_n * rank * hidden, dtype=torch.float32).reshape(e_n * rank, hidden) + 200
    d_b = torch.arange(inter * e_n * rank, dtype=torch.float32).reshape(inter, e_n * rank) + 300
    t = {f"{PREFIX}.base_layer.lora_A.weight": gu_a, f"{PREFIX}.base_layer.lora_B.weight": gu_b,
         f"{PREFIX}.lora_A.weight": d_a, f"{PREFIX}.lora_B.weight": d_b}
    out, _ = A.to_vllm_lora_tensors(t, adapter_config={"r": rank})
    expected = {}
    for e in range(e_n):
        rows = slice(e * rank, (e + 1) * rank)
        gate_a, up_a = gu_a[rows].split(inter, dim=1)
        p = f"{PREFIX}.{e}"
        expected[f"{p}.gate_proj.lora_A.weight"] = gu_b[:, rows].T.contiguous()
        expected[f"{p}.gate_proj.lora_B.weight"] = gate_a.T.contiguous()
        expected[f"{p}.up_proj.lora_A.weight"] = gu_b[:, rows].T.contiguous()
        expected[f"{p}.up_proj.lora_B.weight"] = up_a.T.contiguous()
        expected[f"{p}.down_proj.lora_A.weight"] = d_b[:, rows].T.contiguous()
        expected[f"{p}.down_proj.lora_B.weight"] = d_a[rows].T.contiguous()
    _assert_same(out, expected)


def test_passthrough_and_errors():
    per_expert = {f"{PREFIX}.0.gate_proj.lora_A.weight": torch.zeros(2, 3)}
    out, cfg = A.to_vllm_lora_tensors(per_expert, adapter_config={"target_modules": ["q_proj"]})
    assert out is per_expert and cfg["target_modules"] == ["q_proj", "experts"]
    dense = {"x.q_proj.lora_A.weight": torch.zeros(2, 3)}
    out, cfg = A.to_vllm_lora_tensors(dense, adapter_config={"target_modules": ["q_proj"]})
    assert out is dense and cfg == {"target_modules": ["q_proj"]}
    fused, _ = _fused_fixture()
    del fused[f"{PREFIX}.lora_B.weight"]
    with pytest.raises(RuntimeError, match="Incomplete"):
        A.to_vllm_lora_tensors(fused, adapter_config={"r": 2})
    fused, _ = _fused_fixture()
    with pytest.raises(RuntimeError, match="divisible"):
        A.to_vllm_lora_tensors(fused, adapter_config={"r": 3})


def _loras(e_n=3, h=16, f=12, r=(4, 4, 4), alpha=8, offset=0, seed=0):
    torch.manual_seed(seed)
    mk = lambda name, i, o, rk: LoRA(f"{PREFIX}.{{expert}}.{name}", i, o, rk, alpha * rk / r[0],
                                     torch.float32, "cpu", num_local_experts=e_n, expert_offset=offset)
    g, u, d = mk("gate_proj", h, f, r[0]), mk("up_proj", h, f, r[1]), mk("down_proj", f, h, r[2])
    with torch.no_grad():
        for m in (g, u, d):
            m.B_T.normal_(0, 0.1)
    return g, u, d


def _delta(lora, e):
    """The expert's weight delta scale * B A as [out, in]."""
    return lora.scale * lora.B_T[e].detach().T @ lora.A_T[e].detach().T


def test_megatron_pair_export_applies_the_same_adapter():
    g, u, d = _loras(offset=5)
    w = A.grouped_moe_adapter_weights("decoder.layers.0", g, u, d)
    assert sorted(w) == sorted([f"decoder.layers.0.mlp.experts.linear_fc1.weight{e}" for e in (5, 6, 7)]
                               + [f"decoder.layers.0.mlp.experts.linear_fc2.weight{e}" for e in (5, 6, 7)])
    for e in range(3):
        (pair,) = w[f"decoder.layers.0.mlp.experts.linear_fc1.weight{e + 5}"]
        assert pair.dim == 8 and pair.alpha == 16 and pair.adapter_key is None
        assert pair.linear_in_name == "decoder.layers.0.mlp.experts.linear_fc1.adapter.linear_in.weight"
        got = pair.alpha / pair.dim * pair.linear_out @ pair.linear_in
        torch.testing.assert_close(got, torch.cat([_delta(g, e), _delta(u, e)]), rtol=0, atol=1e-6)
        (down,) = w[f"decoder.layers.0.mlp.experts.linear_fc2.weight{e + 5}"]
        assert down.dim == 4 and down.alpha == 8
        torch.testing.assert_close(down.alpha / down.dim * down.linear_out @ down.linear_in,
                                   _delta(d, e), rtol=0, atol=1e-6)


def test_fused_export_of_art_factors_round_trips_through_the_expander():
    """ART factors -> fused 2D block (pair rank 2r, down zero-padded) ->
    per-expert tensors: every expert's gate, up and down maps are unchanged."""
    g, u, d = _loras(r=(4, 4, 3))
    tensors, rank, alpha = A.fused_moe_lora_tensors(g, u, d, PREFIX)
    assert rank == 8
    out, cfg = A.to_vllm_lora_tensors(tensors, adapter_config={"r": rank, "lora_alpha": alpha})
    s = alpha / rank
    for e in range(3):
        p = f"{PREFIX}.{e}"
        for name, lora in (("gate_proj", g), ("up_proj", u), ("down_proj", d)):
            got = s * out[f"{p}.{name}.lora_B.weight"] @ out[f"{p}.{name}.lora_A.weight"]
            torch.testing.assert_close(got, _delta(lora, e), rtol=0, atol=1e-6)
    assert "experts" in cfg["target_modules"]


def test_per_expert_tensors_round_trip_into_modules():
    g, u, d = _loras(seed=1)
    t = A.expert_lora_tensors(g, u, d)
    assert len(t) == 3 * 3 * 2 and t[f"{PREFIX}.1.down_proj.lora_A.weight"].shape == (4, 12)
    g2, u2, d2 = _loras(seed=2)
    A.load_expert_lora_tensors(g2, u2, d2, t)
    for a, b in ((g, g2), (u, u2), (d, d2)):
        assert torch.equal(a.A_T, b.A_T) and torch.equal(a.B_T, b.B_T)


def test_alpha_must_be_integral():
    lora = LoRA(f"{PREFIX}.{{expert}}.gate_proj", 8, 8, 3, 1.0, torch.float32, "cpu", num_local_experts=2)
    assert A.adapter_alpha_dim(lora) == (1, 3)
    lora.scale = 0.3   # alpha 0.9
    with pytest.raises(ValueError, match="integer alpha"):
        A.adapter_alpha_dim(lora)


def _dense_modules(seed=0):
    from art_amd.megatron.dense_lora import (SelfAttentionLinearProjLoRA, SelfAttentionLinearQKVLoRA,
                                             SharedExpertsLinearFC1LoRA, SharedExpertsLinearFC2LoRA)
    g = torch.Generator().manual_seed(seed)
    qkv = SelfAttentionLinearQKVLoRA("l.self_attn", torch.zeros(2 * (32 + 32), 64, dtype=torch.bfloat16),
                                     4, 8, num_attention_heads=4, num_query_groups=2, kv_channels=16)
    proj = SelfAttentionLinearProjLoRA("l.self_attn.o_proj", torch.zeros(64, 64, dtype=torch.bfloat16), 4, 8)
    fc1 = SharedExpertsLinearFC1LoRA("l.mlp", torch.zeros(96, 64, dtype=torch.bfloat16), 4, 8)
    fc2 = SharedExpertsLinearFC2LoRA("l.mlp", torch.zeros(64, 48, dtype=torch.bfloat16), 4, 8)
    with torch.no_grad():
        for m in (qkv, proj, fc1, fc2):
            for p in m.parameters():
                p.copy_(torch.randn(p.shape, generator=g).to(p.dtype))
    return qkv, proj, fc1, fc2


def test_self_attention_adapter_weights_keys_and_tensors():
    """Attention export (adapter_export.py:236-262): linear_proj plain, linear_qkv
    as adapter_q / adapter_k / adapter_v under one base weight."""
    from types import SimpleNamespace
    qkv, proj, _, _ = _dense_modules()
    out = {}
    A.add_self_attention_adapter_weights(out, layer_prefix="decoder.layers.3",
                                         self_attention=SimpleNamespace(linear_qkv=qkv, linear_proj=proj))
    assert sorted(out) == ["decoder.layers.3.self_attention.linear_proj.weight",
                           "decoder.layers.3.self_attention.linear_qkv.weight"]
    (pw,) = out["decoder.layers.3.self_attention.linear_proj.weight"]
    assert pw.adapter_key is None and (pw.alpha, pw.dim) == (8, 4)
    assert pw.linear_in_name == "decoder.layers.3.self_attention.linear_proj.adapter.linear_in.weight"
    assert torch.equal(pw.linear_in, proj.lora.A_T.detach().t())
    assert torch.equal(pw.linear_out, proj.lora.B_T.detach().t())
    ws = out["decoder.layers.3.self_attention.linear_qkv.weight"]
    assert [w.adapter_key for w in ws] == ["adapter_q", "adapter_k", "adapter_v"]
    assert ws[1].linear_out_name.endswith("linear_qkv.adapter.adapter_k.linear_out.weight")
    for w, lora in zip(ws, (qkv.q_proj_lora, qkv.k_proj_lora, qkv.v_proj_lora)):
        assert torch.equal(w.linear_out, lora.B_T.detach().t())
    assert ws[0].linear_out.shape == (2 * 32, 4) and ws[2].linear_out.shape == (2 * 16, 4)


def test_split_mlp_adapter_weights_match_reference_type_rules():
    """Dense MLP export (adapter_export.py:412-434): gate / up keyed adapters on
    linear_fc1; linear_fc2 only when it is a projection-style linear, so the
    shared-expert FC2 wrapper is skipped exactly as in the reference."""
    from types import SimpleNamespace
    _, proj, fc1, fc2 = _dense_modules(1)
    out = {}
    A.add_split_mlp_adapter_weights(out, "decoder.layers.0.mlp.shared_experts",
                                    SimpleNamespace(linear_fc1=fc1, linear_fc2=fc2))
    assert list(out) == ["decoder.layers.0.mlp.shared_experts.linear_fc1.weight"]
    gate, up = out["decoder.layers.0.mlp.shared_experts.linear_fc1.weight"]
    assert (gate.adapter_key, up.adapter_key) == ("adapter_gate", "adapter_up")
    assert torch.equal(up.linear_in, fc1.up_lora.A_T.detach().t())
    out = {}
    A.add_split_mlp_adapter_weights(out, "decoder.layers.0.mlp",
                                    SimpleNamespace(linear_fc1=fc1, linear_fc2=proj))
    (w2,) = out["decoder.layers.0.mlp.linear_fc2.weight"]
    assert w2.adapter_key is None and torch.equal(w2.linear_out, proj.lora.B_T.detach().t())
