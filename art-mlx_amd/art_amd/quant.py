"""fp8 (OCP e4m3fn) weight storage for the frozen expert weights.

A weight ``W [E, N, K]`` is stored as ``q = e4m3fn(W / s)`` with one fp32
scale per output row, ``s[e, n] = max_k |W[e, n, k]| / 448`` (448 = the
largest e4m3fn value); the dequantised weight is ``bf16(q * s)``, which is
what the products compute with (the fp8-to-bf16 dequantisation of the
reference's fp8 checkpoints, /root/reference/src/art/megatron/dsv4/bridge.py:164-196,
here with per-output-channel instead of block scales).
"""
from __future__ import annotations

import torch

E4M3_MAX = 448.0


def quantize_fp8_rows(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(q float8_e4m3fn [..., N, K], scale fp32 [..., N]) with per-row amax scaling."""
    wf = w.float()
    amax = wf.abs().amax(dim=-1)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (wf / scale.unsqueeze(-1)).to(torch.float8_e4m3fn)
    return q.contiguous(), scale.contiguous()


def dequantize_fp8_rows(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16(q * scale): the weight the fp8 products use."""
    return (q.float() * scale.unsqueeze(-1)).to(torch.bfloat16)


def transpose_fp8(q: torch.Tensor) -> torch.Tensor:
    """[E, N, K] -> [E, K, N] copy of fp8 bytes (the data-gradient operand)."""
    return q.view(torch.uint8).transpose(1, 2).contiguous().view(torch.float8_e4m3fn)
