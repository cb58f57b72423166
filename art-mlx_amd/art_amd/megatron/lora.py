"""LoRA modules of ART's Megatron backend on the HIP grouped products.

Mirrors the module surface of /root/reference/src/art/megatron/lora.py for the
expert path:

* ``LoRA`` (lora.py:451-835): ``A_T [E, in, r]`` / ``B_T [E, r, out]``
  (the expert dimension squeezed for one expert), ``scale = alpha / rank``,
  A Kaiming-uniform(a=sqrt(5)) per expert on ``A_T[e].T`` and B zero
  (PEFT defaults, :529-538), ``forward(x, tokens_per_expert=None)`` with the
  grouped path for several experts and zeros for empty input (:817-835), and
  the adapter export ``{prefix.format(expert=e)}.lora_A.weight = A_T[e].T``
  (:741-786).
* ``GroupedLinear``: the frozen TE grouped linear the LoRA wrappers sit on
  (``forward(x, m_splits) -> (out, None)``, per-expert ``weight{e} [out, in]``,
  lora.py:1097-1100); bf16 or fp8 e4m3fn weights.
* ``MLPExpertsLinearFC1LoRA`` / ``MLPExpertsLinearFC2LoRA`` (lora.py:1464-1571):
  base grouped product plus gate/up (dual, shared projection) or down LoRA.
* ``GroupedMLP``: ``forward(permuted_local_hidden_states, tokens_per_expert,
  permuted_probs)`` of megatron's TEGroupedMLP (signature
  tests/integration/megatron/routing_replay/trace.py:498-513): FC1 LoRA ->
  weighted SwiGLU -> FC2 LoRA.

Not mirrored: multi-adapter slots (``LoRASlotRef``), tensor-parallel sharding
metadata and adapter loading from PEFT checkpoints.  The fused, faster path
for the whole layer is ``moe_layer.moe_lora_layer``.
"""
from __future__ import annotations

import math

import torch

from .. import ops
from .kernels.grouped_lora_hip import quack_grouped_lora, quack_grouped_lora_dual
from .moe_utils import weighted_bias_swiglu_impl

LORA_ALPHA = 32  # lora.py:40


def _counts(tokens_per_expert) -> torch.Tensor:
    if isinstance(tokens_per_expert, list):
        return torch.tensor(tokens_per_expert, dtype=torch.int64, device="cpu")
    return tokens_per_expert


class LoRA(torch.nn.Module):
    def __init__(self, adapter_model_prefix: str, in_features: int, out_features: int, rank: int,
                 alpha: float, dtype: torch.dtype, device, num_local_experts: int = 1,
                 expert_offset: int = 0) -> None:
        super().__init__()
        if num_local_experts > 1 and "{expert}" not in adapter_model_prefix:
            raise ValueError("adapter_model_prefix must contain the '{expert}' format "
                             "placeholder if num_local_experts > 1")
        self.adapter_model_prefix = adapter_model_prefix
        self.alpha = float(alpha)
        self.in_features, self.out_features = int(in_features), int(out_features)
        self.scale = alpha / rank
        self._expert_offset = int(expert_offset)
        self.A_T = torch.nn.Parameter(
            torch.zeros(num_local_experts, in_features, rank, dtype=dtype, device=device).squeeze(0))
        self.B_T = torch.nn.Parameter(
            torch.zeros(num_local_experts, rank, out_features, dtype=dtype, device=device).squeeze(0))
        self.reset_lora_parameters()

    @property
    def num_local_experts(self) -> int:
        return self.A_T.shape[0] if self.A_T.ndim == 3 else 1

    def reset_lora_parameters(self) -> None:
        """A Kaiming-uniform(a=sqrt(5)) on each expert's [rank, in] view, B zero."""
        with torch.no_grad():
            if self.A_T.ndim == 3:
                for e in range(self.A_T.shape[0]):
                    torch.nn.init.kaiming_uniform_(self.A_T[e].T, a=math.sqrt(5))
            else:
                torch.nn.init.kaiming_uniform_(self.A_T.T, a=math.sqrt(5))
            self.B_T.zero_()

    def forward(self, x: torch.Tensor, tokens_per_expert=None) -> torch.Tensor:
        if tokens_per_expert is not None:
            if self.num_local_experts <= 1:
                raise ValueError("tokens_per_expert is only supported if num_local_experts > 1")
            if x.shape[0] == 0:
                return x.new_zeros((*x.shape[:-1], self.out_features))
            return quack_grouped_lora(x, self.A_T, self.B_T, _counts(tokens_per_expert),
                                      scale=self.scale)
        out = (x @ self.A_T) @ self.B_T
        return out if self.scale == 1.0 else out * self.scale

    def _keys(self, expert: int | None, suffix: str) -> str:
        if expert is None:
            return f"{self.adapter_model_prefix}.{suffix}"
        return f"{self.adapter_model_prefix.format(expert=expert + self._expert_offset)}.{suffix}"

    def sharded_lora_state_dict(self) -> dict[str, torch.Tensor]:
        """PEFT layout: lora_A.weight = A_T[e].T [r, in], lora_B.weight = B_T[e].T [out, r]."""
        out: dict[str, torch.Tensor] = {}
        experts = range(self.num_local_experts) if self.A_T.ndim == 3 else [None]
        for e in experts:
            a = self.A_T.data[e] if e is not None else self.A_T.data
            b = self.B_T.data[e] if e is not None else self.B_T.data
            out[self._keys(e, "lora_A.weight")] = a.T
            out[self._keys(e, "lora_B.weight")] = b.T
        return out

    def load_lora_state_dict(self, state: dict[str, torch.Tensor]) -> None:
        """Inverse of ``sharded_lora_state_dict``."""
        experts = range(self.num_local_experts) if self.A_T.ndim == 3 else [None]
        with torch.no_grad():
            for e in experts:
                a = state[self._keys(e, "lora_A.weight")].T
                b = state[self._keys(e, "lora_B.weight")].T
                (self.A_T[e] if e is not None else self.A_T).copy_(a)
                (self.B_T[e] if e is not None else self.B_T).copy_(b)


class _GroupedLinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, lin: "GroupedLinear", counts):
        seg = ops.segments_from_counts(counts, lin.num_gemms, x.device)
        ctx.lin, ctx.seg = lin, seg
        return ops.grouped_gemm(x.contiguous(), lin.weight, seg, lin.num_gemms,
                                b_scale=lin.weight_scale)

    @staticmethod
    def backward(ctx, dy):
        lin, seg = ctx.lin, ctx.seg
        dx = ops.grouped_gemm(dy.contiguous(), lin.weight_t, seg, lin.num_gemms,
                              b_scale=lin.weight_scale, scale_per_k=True)
        return dx, None, None


class GroupedLinear(torch.nn.Module):
    """Frozen per-expert linear ``y_e = x_e W_e^T`` over contiguous expert
    segments (TE GroupedLinear forward/dgrad; no bias, weights not trained).

    ``weight`` [E, out, in] bf16, or fp8 e4m3fn with ``weight_scale`` [E, out].
    """

    def __init__(self, weight: torch.Tensor, weight_scale: torch.Tensor | None = None) -> None:
        super().__init__()
        from ..quant import transpose_fp8
        self.num_gemms, self.out_features, self.in_features = (int(d) for d in weight.shape)
        self.register_buffer("weight", weight.detach().contiguous())
        self.register_buffer("weight_scale", None if weight_scale is None
                             else weight_scale.detach().float().contiguous())
        wt = transpose_fp8(self.weight) if weight_scale is not None else ops.transposed(self.weight)
        self.register_buffer("weight_t", wt)

    def forward(self, x: torch.Tensor, m_splits):
        if x.shape[0] == 0:
            return x.sum() * 0.0 + x.new_zeros((0, self.out_features)), None
        return _GroupedLinearFn.apply(x, self, _counts(m_splits)), None


class MLPExpertsLinearFC1LoRA(torch.nn.Module):
    def __init__(self, adapter_model_prefix: str, linear_fc1: GroupedLinear, rank: int,
                 alpha: float, num_local_experts: int) -> None:
        super().__init__()
        self.linear_fc1 = linear_fc1
        f = linear_fc1.out_features // 2
        w = linear_fc1.weight
        dtype = torch.bfloat16 if w.dtype != torch.float32 else w.dtype
        kw = dict(rank=rank, alpha=alpha, dtype=dtype, device=w.device,
                  num_local_experts=num_local_experts)
        self.gate_lora = LoRA(f"{adapter_model_prefix}.{{expert}}.gate_proj",
                              linear_fc1.in_features, f, **kw)
        self.up_lora = LoRA(f"{adapter_model_prefix}.{{expert}}.up_proj",
                            linear_fc1.in_features, f, **kw)

    def forward(self, x: torch.Tensor, tokens_per_expert):
        base, bias = self.linear_fc1(x, tokens_per_expert)
        if x.shape[0] == 0:
            return base, bias
        adapter = quack_grouped_lora_dual(
            x, self.gate_lora.A_T, self.gate_lora.B_T, self.up_lora.A_T, self.up_lora.B_T,
            _counts(tokens_per_expert), scale_gate=self.gate_lora.scale,
            scale_up=self.up_lora.scale)
        return base + adapter, bias


class MLPExpertsLinearFC2LoRA(torch.nn.Module):
    def __init__(self, adapter_model_prefix: str, linear_fc2: GroupedLinear, rank: int,
                 alpha: float, num_local_experts: int) -> None:
        super().__init__()
        self.linear_fc2 = linear_fc2
        w = linear_fc2.weight
        dtype = torch.bfloat16 if w.dtype != torch.float32 else w.dtype
        self.lora = LoRA(f"{adapter_model_prefix}.{{expert}}.down_proj", linear_fc2.in_features,
                         linear_fc2.out_features, rank=rank, alpha=alpha, dtype=dtype,
                         device=w.device, num_local_experts=num_local_experts)

    def forward(self, x: torch.Tensor, tokens_per_expert):
        base, bias = self.linear_fc2(x, tokens_per_expert)
        if x.shape[0] == 0:
            return base, bias
        return base + self.lora(x, tokens_per_expert=tokens_per_expert), bias


class GroupedMLP(torch.nn.Module):
    """Expert MLP on permuted tokens: FC1 (+gate/up LoRA) -> weighted SwiGLU ->
    FC2 (+down LoRA), as megatron's TEGroupedMLP with ART's LoRA wrappers."""

    def __init__(self, linear_fc1: MLPExpertsLinearFC1LoRA,
                 linear_fc2: MLPExpertsLinearFC2LoRA) -> None:
        super().__init__()
        self.linear_fc1, self.linear_fc2 = linear_fc1, linear_fc2

    def forward(self, permuted_local_hidden_states: torch.Tensor, tokens_per_expert,
                permuted_probs: torch.Tensor):
        y1, _ = self.linear_fc1(permuted_local_hidden_states, tokens_per_expert)
        h = weighted_bias_swiglu_impl(y1, None, permuted_probs.unsqueeze(-1))
        return self.linear_fc2(h, tokens_per_expert)
