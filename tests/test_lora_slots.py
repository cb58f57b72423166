"""LoRA adapter slots and the drop-in's host-side row check, on the CPU.

Restates the slot behaviour exercised by the reference's
tests/integration/megatron/lora/test_dynamic_lora_slots.py:30-70 (which needs
megatron and CUDA): a base-model ref and a missing slot contribute zeros, a
loaded slot multiplies with its own factors and ``alpha / slot_rank``, and
adapters are loaded from PEFT keys (lora.py:549-600, 804-835).  The single
(non-grouped) forward of ``LoRA`` is plain torch, so it runs here; the grouped
path is covered on the GPU (tests/test_gpu_boundary.py).
"""
import pytest
import torch

from art_amd.megatron.lora import LORA_ALPHA, LoRA, LoRASlotRef, use_lora_slot, \
    with_captured_lora_slot


def _adapter(prefix: str, rank: int, seed: int, d_in=4, d_out=5, experts=None):
    g = torch.Generator().manual_seed(seed)
    keys = [prefix] if experts is None else [prefix.format(expert=e) for e in range(experts)]
    out = {}
    for k in keys:
        out[f"{k}.lora_A.weight"] = torch.randn(rank, d_in, generator=g)
        out[f"{k}.lora_B.weight"] = torch.randn(d_out, rank, generator=g)
    return out


def test_slots_select_factors_scale_and_zeros():
    lora = LoRA("dense", 4, 5, 2, 32, torch.float32, "cpu")
    ref_a, ref_b = LoRASlotRef("checkpoint", "A"), LoRASlotRef("checkpoint", "B")
    assert lora.load_lora_slot(ref_a, _adapter("dense", 1, 1), requires_grad=True)
    assert lora.load_lora_slot(ref_b, _adapter("dense", 4, 2), requires_grad=True)
    x = torch.randn(7, 4)
    with use_lora_slot(LoRASlotRef("checkpoint", None)):
        assert torch.equal(lora(x), torch.zeros(7, 5))
        assert lora.active_lora_tensors() is None
    with use_lora_slot(LoRASlotRef("lora", "missing")):
        assert torch.equal(lora(x), torch.zeros(7, 5))
    slot_a = lora._slot(ref_a)
    assert slot_a.rank == 1 and slot_a.scale == 32.0 and lora._slot(ref_b).scale == 8.0
    with use_lora_slot(ref_a):
        got = lora(x)
    assert torch.allclose(got, (x @ slot_a.A_T) @ slot_a.B_T * 32.0, atol=0, rtol=0)
    # the PEFT tensors land transposed: A_T = lora_A.T, B_T = lora_B.T
    ad = _adapter("dense", 1, 1)
    assert torch.equal(slot_a.A_T.detach(), ad["dense.lora_A.weight"].T)
    assert torch.equal(slot_a.B_T.detach(), ad["dense.lora_B.weight"].T)
    # outside any selection the module's own factors are used
    with torch.no_grad():
        lora.B_T.normal_()
    assert torch.allclose(lora(x), (x @ lora.A_T) @ lora.B_T * lora.scale)
    # nested selections restore the outer one
    with use_lora_slot(ref_a):
        with use_lora_slot(ref_b):
            assert lora.active_lora_tensors()[2] == 8.0
        assert lora.active_lora_tensors()[2] == 32.0
    assert lora.active_lora_tensors()[0] is lora.A_T


def test_slot_gradients_reach_only_the_selected_slot():
    lora = LoRA("dense", 4, 5, 2, 32, torch.float32, "cpu")
    ref = LoRASlotRef("checkpoint", "A")
    lora.load_lora_slot(ref, _adapter("dense", 2, 3), requires_grad=True)
    with use_lora_slot(ref):
        lora(torch.randn(3, 4)).sum().backward()
    a, b = lora.lora_slot_params(ref)
    assert a.grad is not None and b.grad is not None
    assert lora.A_T.grad is None and lora.B_T.grad is None
    # a live slot (grads present) may not be overwritten
    with pytest.raises(RuntimeError, match="Cannot overwrite live LoRA slot"):
        lora.load_lora_slot(ref, _adapter("dense", 2, 4), requires_grad=True)
    a.grad = b.grad = None
    assert lora.load_lora_slot(ref, _adapter("dense", 3, 4), requires_grad=False)
    assert lora._slot(ref).rank == 3 and not lora._slot(ref).A_T.requires_grad


def test_slot_loading_keys_device_dtype_and_export():
    lora = LoRA("m.experts.{expert}.up_proj", 4, 5, 2, LORA_ALPHA, torch.bfloat16, "cpu",
                num_local_experts=3)
    ref = LoRASlotRef("lora", "x")
    assert not lora.load_lora_slot(ref, {"unrelated.lora_A.weight": torch.zeros(1)},
                                   requires_grad=True)
    full = {k: v.double() for k, v in _adapter("m.experts.{expert}.up_proj", 2, 5,
                                                experts=3).items()}
    partial = dict(full)
    partial.pop("m.experts.1.up_proj.lora_B.weight")
    with pytest.raises(KeyError, match="Incomplete LoRA adapter keys"):
        lora.load_lora_slot(ref, partial, requires_grad=True)
    assert lora.load_lora_slot(ref, full, requires_grad=True)
    slot = lora._slot(ref)
    assert slot.A_T.shape == (3, 4, 2) and slot.B_T.shape == (3, 2, 5)
    assert slot.A_T.dtype == torch.bfloat16 and slot.A_T.device == lora.A_T.device
    sd = lora.sharded_lora_state_dict(ref)
    assert set(sd) == set(full)
    for k, v in full.items():
        assert torch.equal(sd[k], v.to(torch.bfloat16))
    assert lora.sharded_lora_state_dict(LoRASlotRef("lora", "absent")) == {}
    with pytest.raises(ValueError, match="base-model slot refs"):
        lora.load_lora_slot(LoRASlotRef("lora", None), full, requires_grad=True)


def test_captured_slot_survives_the_context():
    lora = LoRA("dense", 4, 5, 2, 32, torch.float32, "cpu")
    ref = LoRASlotRef("checkpoint", "A")
    lora.load_lora_slot(ref, _adapter("dense", 2, 6), requires_grad=True)
    x = torch.randn(2, 4)
    with use_lora_slot(ref):
        fn = with_captured_lora_slot(lambda v: lora(v))
        inside = lora(x)
    assert torch.equal(fn(x), inside)            # recompute outside: same slot
    assert not torch.equal(lora(x), inside)      # plain call outside: own factors


def test_fused_gate_up_module_layout():
    from art_amd.megatron.lora import MLPExpertsLinearFC1LoRA

    class _Lin:   # the frozen linear's attributes the wrapper reads
        in_features, out_features = 8, 12
        weight = torch.zeros(3, 12, 8, dtype=torch.bfloat16)

    m = MLPExpertsLinearFC1LoRA("layers.0.mlp.experts", _Lin(), 4, 32, 3, fused_gate_up=True)
    assert m.lora.A_T.shape == (3, 8, 4) and m.lora.B_T.shape == (3, 4, 12)
    assert set(m.lora.sharded_lora_state_dict()) == {
        f"layers.0.mlp.experts.{e}.gate_up_proj.lora_{ab}.weight" for e in range(3) for ab in "AB"}
    d = MLPExpertsLinearFC1LoRA("layers.0.mlp.experts", _Lin(), 4, 32, 3)
    assert d.gate_lora.B_T.shape == (3, 4, 6) and d.up_lora.B_T.shape == (3, 4, 6)


def test_drop_in_rejects_more_rows_than_x_for_host_counts():
    from art_amd.megatron.kernels.grouped_lora_hip import _check_rows
    x = torch.zeros(10, 8)
    _check_rows(torch.tensor([4, 0, 6]), x)
    _check_rows(torch.tensor([4, 0, 5]), x)   # fewer rows than x: the caller's contract
    with pytest.raises(ValueError, match="more than the 10 rows"):
        _check_rows(torch.tensor([4, 1, 6]), x)
