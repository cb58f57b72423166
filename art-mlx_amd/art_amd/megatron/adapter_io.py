"""LoRA adapter layouts of the grouped-MoE expert layer.

Converts between the layouts an expert adapter lives in on its way from the
trainer to inference:

* ART's per-expert factors on the LoRA modules (``A_T [E, in, r]``,
  ``B_T [E, r, out]``, ``scale = alpha / r``; ``lora.LoRA``);
* PEFT per-expert tensors ``{prefix}.{e}.{gate,up,down}_proj.lora_{A,B}.weight``
  (``lora_A [r, in]``, ``lora_B [out, r]``);
* megatron-bridge adapter weights: one ``AdapterWeight`` per expert and base
  weight, the gate and up adapters fused into one pair (stacked ``linear_in``,
  block-diagonal ``linear_out``, rank 2r) — adapter_export.py:105-142, 339-383;
  for the dense linears (attention projection, packed QKV, shared / dense MLP)
  keyed adapters per base weight — adapter_export.py:236-262, 412-434;
* the fused 2D MoE tensors of PEFT target-parameter checkpoints and vLLM's
  fused experts (``mlp.experts.[base_layer.]lora_{A,B}.weight``, experts
  stacked along the rank): expanded to per-expert tensors as the Qwen3-MoE
  handler does (handlers/qwen3_moe.py:82-236) and orientation-swapped from
  PEFT to vLLM as utils/convert_moe_lora.py:35-62 does.

All of it is host-side tensor layout (no kernels); every conversion is exact
(copies, transposes, zero padding).
"""
from __future__ import annotations

import json
import math
import os
import re
from dataclasses import dataclass
from typing import Any

import torch

from .lora import LoRA, MLPExpertsLinearFC1LoRA, MLPExpertsLinearFC2LoRA

# ------------------------------------------------ megatron-bridge adapter weights


@dataclass
class AdapterWeight:
    """One adapter of a base weight in megatron-bridge's export form
    (peft_bridge.AdapterWeight: linear_in [dim, in], linear_out [out, dim],
    effective scale alpha / dim)."""
    global_base_prefix: str
    adapter_key: str | None
    alpha: int
    dim: int
    linear_in_name: str
    linear_in: torch.Tensor
    linear_out_name: str
    linear_out: torch.Tensor


def adapter_alpha_dim(lora: LoRA) -> tuple[int, int]:
    """(alpha, rank) with alpha = scale * rank, an integer (adapter_export.py:22-27)."""
    dim = int(lora.A_T.shape[-1])
    alpha = float(lora.scale) * dim
    rounded = round(alpha)
    if not math.isclose(alpha, rounded):
        raise ValueError(f"LoRA scale {lora.scale} times rank {dim} is not an integer alpha")
    return rounded, dim


def adapter_tensors(lora: LoRA, expert_idx: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(linear_in = A [r, in], linear_out = B [out, r]) of one expert (adapter_export.py:30-36)."""
    a_t = lora.A_T if expert_idx is None else lora.A_T[expert_idx]
    b_t = lora.B_T if expert_idx is None else lora.B_T[expert_idx]
    return a_t.detach().transpose(-1, -2).contiguous(), b_t.detach().transpose(-1, -2).contiguous()


def _adapter_weight(*, base_prefix: str, adapter_key: str | None, alpha: int, dim: int,
                    linear_in: torch.Tensor, linear_out: torch.Tensor) -> AdapterWeight:
    suffix = "" if adapter_key is None else f".{adapter_key}"
    pp = f"{base_prefix}.adapter{suffix}"
    return AdapterWeight(base_prefix, adapter_key, alpha, dim, f"{pp}.linear_in.weight", linear_in,
                         f"{pp}.linear_out.weight", linear_out)


def simple_adapter_weight(base_prefix: str, lora: LoRA, *, adapter_key: str | None = None,
                          expert_idx: int | None = None) -> AdapterWeight:
    """adapter_export.py:68-84."""
    alpha, dim = adapter_alpha_dim(lora)
    lin, lout = adapter_tensors(lora, expert_idx)
    return _adapter_weight(base_prefix=base_prefix, adapter_key=adapter_key, alpha=alpha, dim=dim,
                           linear_in=lin, linear_out=lout)


def fused_pair_adapter_weight(base_prefix: str, first: LoRA, second: LoRA, *,
                              first_expert_idx: int | None = None,
                              second_expert_idx: int | None = None) -> AdapterWeight:
    """Two adapters of one fused base weight ([first; second] output rows) as
    one adapter of rank r1 + r2: linear_in = [A1; A2], linear_out =
    [[B1, 0], [0, B2]], alpha = scale * (r1 + r2) (adapter_export.py:105-142)."""
    in1, out1 = adapter_tensors(first, first_expert_idx)
    in2, out2 = adapter_tensors(second, second_expert_idx)
    if not math.isclose(float(first.scale), float(second.scale)):
        raise ValueError("fused pair adapters need equal scales")
    r1, r2 = int(in1.shape[0]), int(in2.shape[0])
    dim = r1 + r2
    lout = torch.cat([torch.cat([out1, out1.new_zeros((out1.shape[0], r2))], dim=1),
                      torch.cat([out2.new_zeros((out2.shape[0], r1)), out2], dim=1)], dim=0)
    return _adapter_weight(base_prefix=base_prefix, adapter_key=None,
                           alpha=round(float(first.scale) * dim), dim=dim,
                           linear_in=torch.cat([in1, in2], dim=0), linear_out=lout)


def grouped_moe_adapter_weights(layer_prefix: str, gate: LoRA | None, up: LoRA | None,
                                down: LoRA | None) -> dict[str, list[AdapterWeight]]:
    """Per-expert adapter weights of a grouped-MoE layer keyed
    ``{layer_prefix}.mlp.experts.linear_fc{1,2}.weight{global_expert}``
    (adapter_export.py:154-167, 339-383): FC1 as the fused gate|up pair, FC2
    as a simple adapter."""
    out: dict[str, list[AdapterWeight]] = {}
    if gate is not None and up is not None:
        base = f"{layer_prefix}.mlp.experts.linear_fc1"
        for e in range(gate.num_local_experts):
            out[f"{base}.weight{e + gate._expert_offset}"] = [fused_pair_adapter_weight(
                base, gate, up, first_expert_idx=e, second_expert_idx=e)]
    if down is not None:
        base = f"{layer_prefix}.mlp.experts.linear_fc2"
        for e in range(down.num_local_experts):
            out[f"{base}.weight{e + down._expert_offset}"] = [simple_adapter_weight(
                base, down, expert_idx=e)]
    return out


def _set_lora_weights(out: dict[str, list[AdapterWeight]], base_prefix: str,
                      *items: tuple[LoRA | None, str | None]) -> None:
    weights = [simple_adapter_weight(base_prefix, lora, adapter_key=key)
               for lora, key in items if lora is not None]
    if weights:
        out[f"{base_prefix}.weight"] = weights


def add_self_attention_adapter_weights(out: dict[str, list[AdapterWeight]], *, layer_prefix: str,
                                       self_attention: Any) -> None:
    """Adapters of an attention block's dense LoRA linears, added to ``out``
    (weights/adapter_export.py:236-262): ``linear_proj`` / ``out_proj`` as one
    plain adapter, the packed ``linear_qkv`` as keyed adapters ``adapter_q``,
    ``adapter_k``, ``adapter_v`` (those present) under one base weight."""
    from .dense_lora import SelfAttentionLinearProjLoRA, SelfAttentionLinearQKVLoRA
    for attr in ("linear_proj", "out_proj"):
        proj = getattr(self_attention, attr, None)
        if isinstance(proj, SelfAttentionLinearProjLoRA):
            _set_lora_weights(out, f"{layer_prefix}.self_attention.{attr}", (proj.lora, None))
    qkv = getattr(self_attention, "linear_qkv", None)
    if isinstance(qkv, SelfAttentionLinearQKVLoRA):
        _set_lora_weights(out, f"{layer_prefix}.self_attention.linear_qkv",
                          (qkv.q_proj_lora, "adapter_q"), (qkv.k_proj_lora, "adapter_k"),
                          (qkv.v_proj_lora, "adapter_v"))


def add_split_mlp_adapter_weights(out: dict[str, list[AdapterWeight]], base_prefix: str,
                                  mlp: Any) -> None:
    """Adapters of a split (gate / up / down) dense MLP, added to ``out``
    (weights/adapter_export.py:412-434): ``linear_fc1`` as keyed adapters
    ``adapter_gate`` and ``adapter_up``; ``linear_fc2`` as one plain adapter
    when it is a projection-style linear.  The same type test as the
    reference: a ``SharedExpertsLinearFC2LoRA`` wrapper does not match it."""
    from .dense_lora import SelfAttentionLinearProjLoRA, SharedExpertsLinearFC1LoRA
    fc1 = getattr(mlp, "linear_fc1", None)
    if isinstance(fc1, SharedExpertsLinearFC1LoRA):
        _set_lora_weights(out, f"{base_prefix}.linear_fc1", (fc1.gate_lora, "adapter_gate"),
                          (fc1.up_lora, "adapter_up"))
    fc2 = getattr(mlp, "linear_fc2", None)
    if isinstance(fc2, SelfAttentionLinearProjLoRA):
        _set_lora_weights(out, f"{base_prefix}.linear_fc2", (fc2.lora, None))


def module_loras(linear_fc1: MLPExpertsLinearFC1LoRA, linear_fc2: MLPExpertsLinearFC2LoRA
                 ) -> tuple[LoRA, LoRA, LoRA]:
    """(gate, up, down) adapters of the expert MLP's LoRA wrappers."""
    return linear_fc1.gate_lora, linear_fc1.up_lora, linear_fc2.lora


# ------------------------------------------------------ PEFT per-expert tensors


def expert_lora_tensors(gate: LoRA, up: LoRA, down: LoRA) -> dict[str, torch.Tensor]:
    """PEFT per-expert tensors of the layer's gate, up and down adapters."""
    out: dict[str, torch.Tensor] = {}
    for lora in (gate, up, down):
        out.update({k: v.detach().contiguous() for k, v in lora.sharded_lora_state_dict().items()})
    return out


def load_expert_lora_tensors(gate: LoRA, up: LoRA, down: LoRA,
                             tensors: dict[str, torch.Tensor]) -> None:
    """Inverse of ``expert_lora_tensors`` (ranks must match the modules)."""
    for lora in (gate, up, down):
        lora.load_lora_state_dict(tensors)


# ------------------------------------------------ fused 2D MoE LoRA tensors

FUSED_MOE_KEY_RE = re.compile(
    r"^(?P<prefix>.*\.mlp\.experts)\.(?:(?P<base_layer>base_layer)\.)?(?P<lora>lora_[AB])\.weight$")
EXPERT_MOE_KEY_RE = re.compile(
    r"^.*\.mlp\.experts\.\d+\.(?:gate_proj|up_proj|down_proj)\.lora_[AB]\.weight$")


def pack_lora_b_by_expert(blocks: list[torch.Tensor]) -> torch.Tensor:
    """Per-expert B [out, r] blocks -> the fused [out, r * E] tensor, column
    i * E + e holding expert e's rank column i (inverse of
    ``packed_lora_b_by_expert``)."""
    stacked = torch.stack(blocks, dim=0)
    return stacked.permute(1, 2, 0).reshape(stacked.shape[1], -1).contiguous()


def packed_lora_b_by_expert(tensor: torch.Tensor, *, num_experts: int, rank: int) -> torch.Tensor:
    """Fused [out, r * E] -> [E, out, r] (handlers/qwen3_moe.py:82-88)."""
    return tensor.reshape(tensor.shape[0], rank, num_experts).permute(2, 0, 1)


def expand_fused_moe_lora(prefix: str, slots: dict[str, torch.Tensor], *,
                          rank: int) -> dict[str, torch.Tensor]:
    """Fused MoE LoRA tensors of one ``mlp.experts`` prefix -> per-expert PEFT
    tensors (handlers/qwen3_moe.py:95-200).  ``slots`` maps
    ``base_layer.lora_A``, ``base_layer.lora_B`` (gate|up) and ``lora_A``,
    ``lora_B`` (down).  Two orientations are recognised by their shapes: the
    PEFT target-parameter one (A/B swapped: gate_up A [E r, 2F], B [H, E r];
    down A [E r, H], B [F, E r]) and the standard one (gate_up A [E r, H],
    B [2F, r E] packed by ``pack_lora_b_by_expert``; down A [E r, F],
    B [H, r E]).  Gate and up share the expert's A."""
    try:
        gu_a, gu_b = slots["base_layer.lora_A"], slots["base_layer.lora_B"]
        d_a, d_b = slots["lora_A"], slots["lora_B"]
    except KeyError as exc:
        raise RuntimeError(f"Incomplete MoE LoRA block for {prefix}") from exc
    if any(t.ndim != 2 for t in (gu_a, gu_b, d_a, d_b)):
        raise RuntimeError(f"MoE LoRA tensors for {prefix} must be 2D")
    if gu_a.shape[0] % rank:
        raise RuntimeError(f"{prefix}: gate/up lora_A shape {tuple(gu_a.shape)} is not divisible "
                           f"by rank {rank}")
    e_n = gu_a.shape[0] // rank
    er = e_n * rank
    out: dict[str, torch.Tensor] = {}
    if (gu_b.shape[1] == er and d_b.shape[1] == er and gu_a.shape[1] == 2 * d_b.shape[0]
            and tuple(d_a.shape) == (er, gu_b.shape[0])):
        f = d_b.shape[0]
        for e in range(e_n):
            rows = slice(e * rank, (e + 1) * rank)
            gate_a, up_a = gu_a[rows].split(f, dim=1)
            p = f"{prefix}.{e}"
            out[f"{p}.gate_proj.lora_A.weight"] = gu_b[:, rows].T.contiguous()
            out[f"{p}.gate_proj.lora_B.weight"] = gate_a.T.contiguous()
            out[f"{p}.up_proj.lora_A.weight"] = gu_b[:, rows].T.contiguous()
            out[f"{p}.up_proj.lora_B.weight"] = up_a.T.contiguous()
            out[f"{p}.down_proj.lora_A.weight"] = d_b[:, rows].T.contiguous()
            out[f"{p}.down_proj.lora_B.weight"] = d_a[rows].T.contiguous()
        return out
    if gu_b.shape[0] % 2:
        raise RuntimeError(f"{prefix}: gate/up lora_B rows {gu_b.shape[0]} are not even")
    f = gu_b.shape[0] // 2
    if gu_b.shape[1] != er:
        raise RuntimeError(f"{prefix}: gate/up lora_B shape {tuple(gu_b.shape)} does not match "
                           f"{e_n} experts at rank {rank}")
    if tuple(d_a.shape) != (er, f):
        raise RuntimeError(f"{prefix}: down lora_A shape {tuple(d_a.shape)} does not match "
                           f"expected {(er, f)}")
    if d_b.shape[1] != er:
        raise RuntimeError(f"{prefix}: down lora_B shape {tuple(d_b.shape)} does not match "
                           f"{e_n} experts at rank {rank}")
    gu_be = packed_lora_b_by_expert(gu_b, num_experts=e_n, rank=rank)
    d_be = packed_lora_b_by_expert(d_b, num_experts=e_n, rank=rank)
    for e in range(e_n):
        rows = slice(e * rank, (e + 1) * rank)
        gate_b, up_b = gu_be[e].split(f, dim=0)
        p = f"{prefix}.{e}"
        out[f"{p}.gate_proj.lora_A.weight"] = gu_a[rows].clone()
        out[f"{p}.gate_proj.lora_B.weight"] = gate_b.contiguous()
        out[f"{p}.up_proj.lora_A.weight"] = gu_a[rows].clone()
        out[f"{p}.up_proj.lora_B.weight"] = up_b.contiguous()
        out[f"{p}.down_proj.lora_A.weight"] = d_a[rows].clone()
        out[f"{p}.down_proj.lora_B.weight"] = d_be[e].contiguous()
    return out


def moe_lora_config(adapter_config: dict[str, Any]) -> dict[str, Any]:
    """Adapter config with ``experts`` among the target modules
    (handlers/qwen3_moe.py:73-79)."""
    config = dict(adapter_config)
    targets = list(config.get("target_modules") or [])
    if "experts" not in targets:
        targets.append("experts")
    config["target_modules"] = targets
    return config


def to_vllm_lora_tensors(tensors: dict[str, torch.Tensor], *, adapter_config: dict[str, Any]
                         ) -> tuple[dict[str, torch.Tensor], dict[str, Any]]:
    """Expand every fused ``mlp.experts`` block to per-expert tensors, keep
    the rest (handlers/qwen3_moe.py:203-236)."""
    grouped: dict[str, dict[str, torch.Tensor]] = {}
    for key, t in tensors.items():
        m = FUSED_MOE_KEY_RE.match(key)
        if m is None:
            continue
        slot = f"{'base_layer.' if m.group('base_layer') else ''}{m.group('lora')}"
        grouped.setdefault(m.group("prefix"), {})[slot] = t
    if not grouped:
        if any(EXPERT_MOE_KEY_RE.match(k) for k in tensors):
            return tensors, moe_lora_config(adapter_config)
        return tensors, adapter_config
    rank = int(adapter_config["r"])
    out: dict[str, torch.Tensor] = {}
    used: set[str] = set()
    for prefix, slots in grouped.items():
        out.update(expand_fused_moe_lora(prefix, slots, rank=rank))
        used.update({f"{prefix}.base_layer.lora_A.weight", f"{prefix}.base_layer.lora_B.weight",
                     f"{prefix}.lora_A.weight", f"{prefix}.lora_B.weight"})
    for key, t in tensors.items():
        if key in used:
            continue
        if key in out:
            raise RuntimeError(f"Duplicate LoRA tensor after conversion: {key}")
        out[key] = t
    return out, moe_lora_config(adapter_config)


def fused_moe_lora_tensors(gate: LoRA, up: LoRA, down: LoRA, prefix: str
                           ) -> tuple[dict[str, torch.Tensor], int, int]:
    """The layer's adapters as one fused 2D block in the standard orientation
    (``to_vllm_lora_tensors`` expands it back), with (rank, alpha) for the
    adapter config.  The fused layout has one A per expert shared by gate and
    up, so each expert's gate|up adapter is the fused pair of rank
    r_g + r_u, and the down adapter is zero-padded to the same rank (exact:
    zero rows of A meet zero columns of B)."""
    g, u, d = gate, up, down
    if not (math.isclose(float(g.scale), float(u.scale)) and math.isclose(float(g.scale),
                                                                          float(d.scale))):
        raise ValueError("fused MoE LoRA export needs equal scales on gate, up and down")
    rank = int(g.A_T.shape[-1]) + int(u.A_T.shape[-1])
    rd = int(d.A_T.shape[-1])
    if rd > rank:
        raise ValueError(f"down rank {rd} exceeds the gate|up pair rank {rank}")
    gu_a, gu_b, d_a, d_b = [], [], [], []
    for e in range(g.num_local_experts):
        pair = fused_pair_adapter_weight(prefix, g, u, first_expert_idx=e, second_expert_idx=e)
        gu_a.append(pair.linear_in)
        gu_b.append(pair.linear_out)
        din, dout = adapter_tensors(d, e)
        d_a.append(torch.cat([din, din.new_zeros((rank - rd, din.shape[1]))], dim=0))
        d_b.append(torch.cat([dout, dout.new_zeros((dout.shape[0], rank - rd))], dim=1))
    tensors = {
        f"{prefix}.base_layer.lora_A.weight": torch.cat(gu_a, dim=0).contiguous(),
        f"{prefix}.base_layer.lora_B.weight": pack_lora_b_by_expert(gu_b),
        f"{prefix}.lora_A.weight": torch.cat(d_a, dim=0).contiguous(),
        f"{prefix}.lora_B.weight": pack_lora_b_by_expert(d_b),
    }
    return tensors, rank, round(float(g.scale) * rank)


# ------------------------------------------- PEFT fused checkpoint -> vLLM


def has_peft_fused_moe_lora(tensors: dict[str, torch.Tensor], adapter_config: dict) -> bool:
    """utils/convert_moe_lora.py:21-32."""
    if not adapter_config.get("target_parameters"):
        return False
    return any(re.search(r"mlp\.experts\.(base_layer\.)?lora_[AB]\.weight$", k) for k in tensors)


def convert_fused_moe_lora(tensors: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """PEFT fused MoE LoRA (A/B swapped) -> vLLM's fused orientation: every
    fused A/B pair is swapped and transposed (utils/convert_moe_lora.py:35-62)."""
    out: dict[str, torch.Tensor] = {}
    swap = {"base_layer.lora_A": "base_layer.lora_B", "base_layer.lora_B": "base_layer.lora_A",
            "lora_A": "lora_B", "lora_B": "lora_A"}
    for key, t in tensors.items():
        m = re.match(r"(.*\.mlp\.experts)\.(base_layer\.lora_(A|B)|lora_(A|B))\.weight$", key)
        if not m:
            out[key] = t
            continue
        out[f"{m.group(1)}.{swap[m.group(2)]}.weight"] = t.T.contiguous()
    return out


def convert_checkpoint_if_needed(checkpoint_dir: str) -> bool:
    """Rewrite ``adapter_model.safetensors`` / ``adapter_config.json`` of a PEFT
    fused MoE checkpoint in vLLM's orientation, ``experts`` as the target
    module (utils/convert_moe_lora.py:65-100).  Returns whether it converted."""
    import safetensors.torch
    path = os.path.join(checkpoint_dir, "adapter_model.safetensors")
    cfg_path = os.path.join(checkpoint_dir, "adapter_config.json")
    if not (os.path.exists(path) and os.path.exists(cfg_path)):
        return False
    tensors = safetensors.torch.load_file(path)
    with open(cfg_path) as f:
        config = json.load(f)
    if not has_peft_fused_moe_lora(tensors, config):
        return False
    safetensors.torch.save_file(convert_fused_moe_lora(tensors), path)
    config["target_modules"] = [m for m in config.get("target_modules", [])
                                if m not in {"experts", "gate_proj", "up_proj", "down_proj"}]
    config["target_modules"].append("experts")
    config.pop("target_parameters", None)
    with open(cfg_path, "w") as f:
        json.dump(config, f, indent=2)
    return True
