"""Top-k softmax router with megatron's ``TopKRouter`` surface on the HIP kernels.

The reference trains Qwen3-MoE routers through megatron's ``TopKRouter``:
``gating`` (fp32 router linear, bridge_runtime.py:775-798, provider.py:605)
then ``routing(logits) -> (probs [T,E] fp32, routing_map [T,E] bool)`` with
softmax scores, top-k and renormalisation over the k selected (Qwen3
``norm_topk_prob``; restated in dsv4/layer.py:139-191 and the test fake of
tests/unit/test_moe_routing_replay.py:181-205), where a ``RouterReplay``
target replaces top-k selection (routing_replay.py:1430-1434).

Here ``gating`` is the bf16-MFMA GEMM with fp32 accumulation and fp32 output,
``routing`` the top-k softmax or replay kernel.  ``routing_compact`` returns
the compact ``(idx [T,k], w [T,k], status)`` form the fused expert layer
consumes; ``routing`` expands it to the dense megatron form and carries the
softmax backward to the logits.
"""
from __future__ import annotations

import types

import torch

from .. import ops
from .moe_layer import router_logits
from .routing_replay import RouterReplay


class _RouteFn(torch.autograd.Function):
    """w = softmax over the selected logits; dlogits scatters w (dw - <w, dw>)."""

    @staticmethod
    def forward(ctx, logits, target, k: int):
        if target is None:
            idx, w = ops.router_topk(logits, k)
            status = None
        else:
            idx, w, status = ops.router_replay(logits, target)
        ctx.save_for_backward(idx, w)
        ctx.num_experts = logits.shape[1]
        ctx.mark_non_differentiable(idx)
        if status is not None:
            ctx.mark_non_differentiable(status)
        return w, idx, status

    @staticmethod
    def backward(ctx, dw, _didx, _dstatus):
        idx, w = ctx.saved_tensors
        dl = w * (dw - (w * dw).sum(dim=1, keepdim=True))
        dl = torch.where(idx >= 0, dl, torch.zeros_like(dl))
        dlogits = torch.zeros((w.shape[0], ctx.num_experts), dtype=torch.float32, device=w.device)
        dlogits.scatter_add_(1, idx.clamp_min(0).long(), dl)
        return dlogits, None, None


class _GatingFn(torch.autograd.Function):
    """logits = x W_r^T in fp32; dx = dlogits W_r (router weight frozen)."""

    @staticmethod
    def forward(ctx, x, weight):
        ctx.save_for_backward(weight)
        return router_logits(x, weight)

    @staticmethod
    def backward(ctx, dlogits):
        (weight,) = ctx.saved_tensors
        return (dlogits @ weight.float()).to(weight.dtype), None


class TopKRouter(torch.nn.Module):
    """Softmax top-k router (renormalised over the k selected)."""

    def __init__(self, hidden_size: int, num_experts: int, topk: int, *,
                 moe_enable_routing_replay: bool = False, sequence_parallel: bool = False,
                 dtype: torch.dtype = torch.bfloat16, device=None, init_std: float = 0.02):
        super().__init__()
        if not 1 <= topk <= num_experts:
            raise ValueError(f"topk must be in [1, num_experts], got {topk} for {num_experts}")
        self.topk = int(topk)
        self.num_experts = int(num_experts)
        w = torch.empty((num_experts, hidden_size), dtype=dtype, device=device)
        torch.nn.init.normal_(w, std=init_std)
        self.weight = torch.nn.Parameter(w, requires_grad=False)
        self.config = types.SimpleNamespace(
            moe_router_fusion=False, sequence_parallel=sequence_parallel, context_parallel_size=1,
            moe_router_topk=self.topk, num_moe_experts=self.num_experts)
        self.router_replay = RouterReplay() if moe_enable_routing_replay else None
        self.last_status: torch.Tensor | None = None

    def gating(self, x: torch.Tensor) -> torch.Tensor:
        return _GatingFn.apply(x.reshape(-1, x.shape[-1]), self.weight)

    def _target(self) -> torch.Tensor | None:
        return self.router_replay.active_target() if self.router_replay is not None else None

    def routing_compact(self, logits: torch.Tensor):
        """(idx int32 [T,k], w fp32 [T,k], status) without autograd; ``status``
        counts rejected replay ids (None without a replay target)."""
        target = self._target()
        if target is None:
            idx, w = ops.router_topk(logits, self.topk)
            status = None
        else:
            idx, w, status = ops.router_replay(logits, target)
        self.last_status = status
        return idx, w, status

    def routing(self, logits: torch.Tensor):
        """(probs [T,E] fp32, routing_map [T,E] bool), differentiable in ``logits``."""
        target = self._target()
        w, idx, status = _RouteFn.apply(logits, target, self.topk)
        self.last_status = status
        t = logits.shape[0]
        cols = idx.long().clamp_min(0)
        keep = idx >= 0
        # scatter-add: a rejected slot (id -1, parked on column 0 with value 0)
        # must not overwrite a selected column 0
        probs = torch.zeros((t, self.num_experts), dtype=torch.float32, device=logits.device)
        probs = probs.scatter_add(1, cols, torch.where(keep, w, torch.zeros_like(w)))
        hits = torch.zeros((t, self.num_experts), dtype=torch.int32, device=logits.device)
        routing_map = hits.scatter_add_(1, cols, keep.to(torch.int32)) > 0
        return probs, routing_map

    def forward(self, x: torch.Tensor):
        return self.routing(self.gating(x))
