"""Grouped (varlen-M) LoRA operator on gfx950 HIP kernels.

Drop-in for ``art.megatron.kernels.cute_grouped_lora_quack``
(/root/reference/src/art/megatron/kernels/cute_grouped_lora_quack.py): same
function names, arguments, validation errors, autograd behaviour and
return dtypes.  Differences are internal:

* offsets never leave the device (segment table built by a kernel from the
  counts, /root/reference/.../cute_grouped_lora_quack.py:97-121 builds them on
  the host);
* ranks are zero-padded to a multiple of 16 (the MFMA K step) instead of to 8
  (:15-25, 205-224) -- padding columns are exact zeros, so results and
  gradients of the true rank are unchanged;
* weight gradients are accumulated in fp32 by a deterministic segmented
  kernel and returned in the parameter dtype, as the reference returns them.
"""
from __future__ import annotations

from typing import Any

import torch

from ... import ops

_PADDED_LOW_RANK_TARGET = 8
_MFMA_K = 16


def _validate_rank(rank: int) -> None:
    # cute_grouped_lora_quack.py:18-25
    if rank <= 0:
        raise ValueError(f"Grouped LoRA HIP backend requires rank > 0, got {rank}")
    if rank >= _PADDED_LOW_RANK_TARGET and rank % _PADDED_LOW_RANK_TARGET != 0:
        raise ValueError(
            "Grouped LoRA HIP backend requires rank < 8 or a multiple of 8, "
            f"got {rank}")


def _tokens_per_expert_to_tensor(tokens_per_expert) -> torch.Tensor:
    # cute_grouped_lora_quack.py:97-106
    if isinstance(tokens_per_expert, list):
        return torch.tensor(tokens_per_expert, dtype=torch.int64, device="cpu")
    if tokens_per_expert.ndim != 1:
        raise ValueError(
            f"tokens_per_expert must be 1D, got shape {tuple(tokens_per_expert.shape)}")
    return tokens_per_expert.detach().to(dtype=torch.int64).contiguous()


def _validate_inputs(x, a_t, b_t, tokens_per_expert) -> torch.Tensor:
    # cute_grouped_lora_quack.py:124-163
    counts = _tokens_per_expert_to_tensor(tokens_per_expert)
    if x.ndim != 2:
        raise ValueError(f"x must be 2D, got shape {tuple(x.shape)}")
    if a_t.ndim != 3:
        raise ValueError(f"a_t must be 3D, got shape {tuple(a_t.shape)}")
    if b_t.ndim != 3:
        raise ValueError(f"b_t must be 3D, got shape {tuple(b_t.shape)}")
    rank = a_t.shape[-1]
    _validate_rank(rank)
    if b_t.shape[-2] != rank:
        raise ValueError(f"Expected b_t rank dim {rank}, got shape {tuple(b_t.shape)}")
    if a_t.shape[0] != b_t.shape[0]:
        raise ValueError(
            "a_t and b_t must have the same number of experts, "
            f"got {a_t.shape[0]} and {b_t.shape[0]}")
    if a_t.shape[1] != x.shape[1]:
        raise ValueError(
            f"a_t input dim must match x.shape[1], got {a_t.shape[1]} and {x.shape[1]}")
    if counts.numel() != a_t.shape[0]:
        raise ValueError(
            "tokens_per_expert length must match number of experts, "
            f"got {counts.numel()} and {a_t.shape[0]}")
    if x.device.type != "cuda" or a_t.device != x.device or b_t.device != x.device:
        raise ValueError("x, a_t, and b_t must be CUDA tensors on the same device")
    if x.dtype not in {torch.float16, torch.bfloat16}:
        raise ValueError(f"Unsupported dtype {x.dtype}; expected fp16 or bf16")
    if a_t.dtype != x.dtype or b_t.dtype != x.dtype:
        raise ValueError(f"Dtype mismatch: x={x.dtype}, a_t={a_t.dtype}, b_t={b_t.dtype}")
    if x.shape[1] % 8 or b_t.shape[-1] % 8:
        raise ValueError("in_features and out_features must be multiples of 8")
    _check_rows(counts, x)
    return counts


def _check_rows(counts: torch.Tensor, x: torch.Tensor) -> None:
    """sum(counts) <= x.shape[0] when the counts are on the host (no sync).

    The reference leaves ``sum(counts) == x.shape[0]`` to the caller
    (cute_grouped_lora_quack.py:642-651).  Host counts cost nothing to check;
    device counts are not read back, and the kernels clamp every segment to
    the rows of x instead."""
    if counts.device.type == "cpu":
        total = int(counts.sum())
        if total > x.shape[0]:
            raise ValueError(
                f"tokens_per_expert sums to {total}, more than the {x.shape[0]} rows of x")


def _validate_dual_inputs(x, gate_a_t, gate_b_t, up_a_t, up_b_t, tokens_per_expert):
    # cute_grouped_lora_quack.py:166-202
    counts = _validate_inputs(x, gate_a_t, gate_b_t, tokens_per_expert)
    if up_a_t.ndim != 3:
        raise ValueError(f"up_a_t must be 3D, got shape {tuple(up_a_t.shape)}")
    if up_b_t.ndim != 3:
        raise ValueError(f"up_b_t must be 3D, got shape {tuple(up_b_t.shape)}")
    up_rank = up_a_t.shape[-1]
    _validate_rank(up_rank)
    if up_b_t.shape[-2] != up_rank:
        raise ValueError(f"Expected up_b_t rank dim {up_rank}, got shape {tuple(up_b_t.shape)}")
    if up_a_t.shape[0] != gate_a_t.shape[0] or up_b_t.shape[0] != gate_b_t.shape[0]:
        raise ValueError(
            "Gate and up tensors must have the same number of experts, "
            f"got gate={gate_a_t.shape[0]} up={up_a_t.shape[0]}")
    if up_a_t.shape[1] != x.shape[1]:
        raise ValueError(
            f"up_a_t input dim must match x.shape[1], got {up_a_t.shape[1]} and {x.shape[1]}")
    if up_a_t.device != x.device or up_b_t.device != x.device:
        raise ValueError("x, up_a_t, and up_b_t must be CUDA tensors on the same device")
    if up_a_t.dtype != x.dtype or up_b_t.dtype != x.dtype:
        raise ValueError(
            f"Dtype mismatch: x={x.dtype}, up_a_t={up_a_t.dtype}, up_b_t={up_b_t.dtype}")
    if up_b_t.shape[-1] % 8:
        raise ValueError("out_features must be multiples of 8")
    return counts


def padded_rank(rank: int) -> int:
    """Rank rounded up to the MFMA K step (16)."""
    return (rank + _MFMA_K - 1) // _MFMA_K * _MFMA_K


def proj_operand(a_ts, ranks_padded) -> torch.Tensor:
    """[E, sum(RP), in]: the A factors transposed and stacked along padded rank."""
    e, d_in = a_ts[0].shape[0], a_ts[0].shape[1]
    out = a_ts[0].new_empty((e, sum(ranks_padded), d_in))
    items, off = [], 0
    for a_t, rp in zip(a_ts, ranks_padded):
        items.append((out[:, off:off + rp], a_t.transpose(1, 2), 1.0))
        off += rp
    ops.pack(*items)
    return out


def apply_operand(b_t: torch.Tensor, rp: int, scale: float = 1.0) -> torch.Tensor:
    """[E, out, RP]: B transposed (optionally scaled), rank zero-padded."""
    e, _r, d_out = b_t.shape
    out = b_t.new_empty((e, d_out, rp))
    ops.pack((out, b_t.transpose(1, 2), scale))
    return out


def pad_rank_last(a_t: torch.Tensor, rp: int) -> torch.Tensor:
    """[E, in, RP] copy of A_T with zero rank padding (A_T itself if already padded)."""
    if a_t.shape[-1] == rp and a_t.is_contiguous():
        return a_t
    out = a_t.new_empty((*a_t.shape[:-1], rp))
    ops.pack((out, a_t, 1.0))
    return out


def pad_rank_mid(b_t: torch.Tensor, rp: int) -> torch.Tensor:
    """[E, RP, out] copy of B_T with zero rank padding (B_T itself if already padded)."""
    if b_t.shape[1] == rp and b_t.is_contiguous():
        return b_t
    out = b_t.new_empty((b_t.shape[0], rp, b_t.shape[2]))
    ops.pack((out, b_t, 1.0))
    return out


def concat_rank_last(a_ts, ranks_padded) -> torch.Tensor:
    """[E, in, sum(RP)]: the A factors side by side, each rank zero-padded."""
    e, d_in = a_ts[0].shape[0], a_ts[0].shape[1]
    out = a_ts[0].new_empty((e, d_in, sum(ranks_padded)))
    items, off = [], 0
    for a_t, rp in zip(a_ts, ranks_padded):
        items.append((out[:, :, off:off + rp], a_t, 1.0))
        off += rp
    ops.pack(*items)
    return out


class _HipGroupedLoraFn(torch.autograd.Function):
    """out = scale * (x_e @ A_T[e]) @ B_T[e]   (cute_grouped_lora_quack.py:337-438)."""

    @staticmethod
    def forward(ctx, x, a_t, b_t, counts, scale):
        e, d_in, r = a_t.shape
        rp = padded_rank(r)
        seg = ops.segments_from_counts(counts, e, x.device)
        x = x.contiguous()
        m = x.shape[0]
        tmp = ops.grouped_gemm(x, proj_operand([a_t], [rp]), seg, e, m=m)
        out = ops.grouped_gemm(tmp, apply_operand(b_t, rp), seg, e, m=m, alpha=scale)
        ctx.save_for_backward(x, a_t, b_t, tmp, seg)
        ctx.scale = scale
        ctx.rp = rp
        return out

    @staticmethod
    def backward(ctx, *grad_outputs: Any):
        x, a_t, b_t, tmp, seg = ctx.saved_tensors
        (grad_out,) = grad_outputs
        assert grad_out.stride(-1) == 1, "HIP grouped LoRA backward requires grad_out stride(-1) == 1"
        grad_out = grad_out.contiguous()
        e, d_in, r = a_t.shape
        rp, scale, m = ctx.rp, ctx.scale, x.shape[0]
        grad_tmp = ops.grouped_gemm(grad_out, pad_rank_mid(b_t, rp), seg, e, m=m, alpha=scale)
        grad_x = ops.grouped_gemm(grad_tmp, pad_rank_last(a_t, rp), seg, e, m=m)
        grad_a = ops.grouped_wgrad(x, grad_tmp, seg, e, out_dtype=a_t.dtype)
        grad_b = ops.grouped_wgrad(grad_out, tmp, seg, e, alpha=scale, transpose_out=True,
                                   out_dtype=b_t.dtype)
        return (grad_x, grad_a[:, :, :r], grad_b[:, :r, :], None, None)


class _HipGroupedLoraDualFn(torch.autograd.Function):
    """[s_g (x A_g) B_g | s_u (x A_u) B_u] with one shared projection
    (cute_grouped_lora_quack.py:441-629)."""

    @staticmethod
    def forward(ctx, x, gate_a_t, gate_b_t, up_a_t, up_b_t, counts, scale_gate, scale_up):
        e = gate_a_t.shape[0]
        rg, ru = gate_a_t.shape[-1], up_a_t.shape[-1]
        rpg, rpu = padded_rank(rg), padded_rank(ru)
        fg, fu = gate_b_t.shape[-1], up_b_t.shape[-1]
        seg = ops.segments_from_counts(counts, e, x.device)
        x = x.contiguous()
        m = x.shape[0]
        tmp = ops.grouped_gemm(x, proj_operand([gate_a_t, up_a_t], [rpg, rpu]), seg, e, m=m)
        out = torch.empty((m, fg + fu), dtype=x.dtype, device=x.device)
        ops.grouped_gemm(tmp[:, :rpg], apply_operand(gate_b_t, rpg), seg, e, m=m,
                         alpha=scale_gate, out=out[:, :fg])
        ops.grouped_gemm(tmp[:, rpg:], apply_operand(up_b_t, rpu), seg, e, m=m,
                         alpha=scale_up, out=out[:, fg:])
        ctx.save_for_backward(x, gate_a_t, gate_b_t, up_a_t, up_b_t, tmp, seg)
        ctx.meta = (rg, ru, rpg, rpu, fg, fu, scale_gate, scale_up)
        return out

    @staticmethod
    def backward(ctx, *grad_outputs: Any):
        x, gate_a_t, gate_b_t, up_a_t, up_b_t, tmp, seg = ctx.saved_tensors
        rg, ru, rpg, rpu, fg, fu, sg, su = ctx.meta
        (grad_out,) = grad_outputs
        assert grad_out.stride(-1) == 1, (
            "HIP grouped FC1 dual LoRA backward requires grad_out stride(-1) == 1")
        grad_out = grad_out.contiguous()
        e, m = gate_a_t.shape[0], x.shape[0]
        grad_tmp = torch.empty((m, rpg + rpu), dtype=x.dtype, device=x.device)
        ops.grouped_gemm(grad_out[:, :fg], pad_rank_mid(gate_b_t, rpg), seg, e, m=m, alpha=sg,
                         out=grad_tmp[:, :rpg])
        ops.grouped_gemm(grad_out[:, fg:], pad_rank_mid(up_b_t, rpu), seg, e, m=m, alpha=su,
                         out=grad_tmp[:, rpg:])
        a_cat = concat_rank_last([gate_a_t, up_a_t], [rpg, rpu])
        grad_x = ops.grouped_gemm(grad_tmp, a_cat, seg, e, m=m)
        grad_a = ops.grouped_wgrad(x, grad_tmp, seg, e, out_dtype=x.dtype)
        grad_bg = ops.grouped_wgrad(grad_out[:, :fg], tmp[:, :rpg], seg, e, alpha=sg,
                                    transpose_out=True, out_dtype=x.dtype)
        grad_bu = ops.grouped_wgrad(grad_out[:, fg:], tmp[:, rpg:], seg, e, alpha=su,
                                    transpose_out=True, out_dtype=x.dtype)
        return (grad_x, grad_a[:, :, :rg], grad_bg[:, :rg, :], grad_a[:, :, rpg:rpg + ru],
                grad_bu[:, :ru, :], None, None, None)


@torch.compiler.disable
def quack_grouped_lora(x, a_t, b_t, counts, scale: float = 1.0) -> torch.Tensor:
    """Grouped LoRA over expert segments (drop-in for the QuACK operator,
    cute_grouped_lora_quack.py:634-654).

    Caller contract (as in the reference): ``counts`` ordered by local expert,
    ``sum(counts) == x.shape[0]`` (not checked: no host sync), ``x`` 2-D,
    ``a_t [E, in, r]``, ``b_t [E, r, out]``, same CUDA device, fp16 or bf16.
    """
    counts_tensor = _validate_inputs(x, a_t, b_t, counts)
    return _HipGroupedLoraFn.apply(x, a_t, b_t, counts_tensor, scale)


@torch.compiler.disable
def quack_grouped_lora_dual(x, gate_a_t, gate_b_t, up_a_t, up_b_t, counts, *,
                            scale_gate: float = 1.0, scale_up: float = 1.0) -> torch.Tensor:
    """Grouped FC1 gate/up LoRA with a shared projection (cute_grouped_lora_quack.py:657-680)."""
    counts_tensor = _validate_dual_inputs(x, gate_a_t, gate_b_t, up_a_t, up_b_t, counts)
    return _HipGroupedLoraDualFn.apply(x, gate_a_t, gate_b_t, up_a_t, up_b_t, counts_tensor,
                                       scale_gate, scale_up)
