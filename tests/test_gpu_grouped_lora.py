"""GPU parity of the drop-in grouped LoRA operators (quack_grouped_lora /
quack_grouped_lora_dual) against the CPU oracle's fp32 per-expert loop.

Mirrors /root/reference/tests/integration/test_lora_quack_cutover.py:69-213:
in = out = 64, E = 4, counts [32, 0, 16, 24] (a zero-token expert), ranks
{1, 3, 7, 16, 24}, seed 20260323 + rank, A/B ~ 0.05 N(0,1), loss
<out, g> / numel; forward, dx, dA, dB at atol = rtol = 5e-2 (the reference's
tolerance) and 2e-2 norm-relative.
"""
import json
from pathlib import Path

import pytest
import torch

from oracle import layer as OL

pytestmark = pytest.mark.gpu
KAT = json.loads((Path(__file__).parent / "golden" / "routing_kats.json").read_text())["lora_cutover"]


def rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _close(got, ref):
    assert rel(got, ref) < 2e-2, rel(got, ref)
    torch.testing.assert_close(got.detach().cpu().float(), ref.detach().float(), atol=5e-2, rtol=5e-2)


@pytest.mark.parametrize("rank", KAT["ranks"])
def test_grouped_lora_matches_oracle(device, rank):
    from art_amd.megatron.kernels.grouped_lora_hip import quack_grouped_lora
    torch.manual_seed(KAT["seed_base"] + rank)
    e, d_in, d_out = len(KAT["counts"]), KAT["in_features"], KAT["out_features"]
    counts = torch.tensor(KAT["counts"], dtype=torch.int64)
    m = int(counts.sum())
    a = (torch.randn(e, d_in, rank) * 0.05).to(torch.bfloat16)
    b = (torch.randn(e, rank, d_out) * 0.05).to(torch.bfloat16)
    x = (torch.randn(m, d_in) * 0.05).to(torch.bfloat16)
    g = torch.randn(m, d_out).to(torch.bfloat16)
    scale = 32 / rank

    xr, ar, br = (v.float().requires_grad_() for v in (x, a, b))
    ref = OL.grouped_lora(xr, ar, br, KAT["counts"], scale)
    ((ref * g.float()).sum() / g.numel()).backward()

    xg = x.to(device).requires_grad_()
    ag = a.to(device).requires_grad_()
    bg = b.to(device).requires_grad_()
    out = quack_grouped_lora(xg, ag, bg, counts, scale=scale)
    ((out.float() * g.to(device).float()).sum() / g.numel()).backward()
    assert out.dtype == torch.bfloat16 and ag.grad.dtype == torch.bfloat16
    _close(out, ref)
    _close(xg.grad, xr.grad)
    _close(ag.grad, ar.grad)
    _close(bg.grad, br.grad)


@pytest.mark.parametrize("rank", KAT["ranks"])
def test_grouped_lora_dual_matches_oracle(device, rank):
    from art_amd.megatron.kernels.grouped_lora_hip import quack_grouped_lora_dual
    torch.manual_seed(KAT["seed_base"] + 1 + rank)
    e, d_in, d_out = len(KAT["counts"]), KAT["in_features"], KAT["out_features"]
    counts = KAT["counts"]
    m = sum(counts)
    mk = lambda *s: (torch.randn(*s) * 0.05).to(torch.bfloat16)
    x, ag_, bg_, au_, bu_ = mk(m, d_in), mk(e, d_in, rank), mk(e, rank, d_out), mk(e, d_in, rank), mk(e, rank, d_out)
    g = torch.randn(m, 2 * d_out).to(torch.bfloat16)
    leaves_ref = [v.float().requires_grad_() for v in (x, ag_, bg_, au_, bu_)]
    ref = OL.grouped_lora_dual(*leaves_ref, counts, 2.0, 3.0)
    ((ref * g.float()).sum() / g.numel()).backward()
    leaves = [v.to(device).requires_grad_() for v in (x, ag_, bg_, au_, bu_)]
    out = quack_grouped_lora_dual(*leaves, counts, scale_gate=2.0, scale_up=3.0)
    ((out.float() * g.to(device).float()).sum() / g.numel()).backward()
    _close(out, ref)
    for got, want in zip(leaves, leaves_ref):
        _close(got.grad, want.grad)


def test_grouped_lora_qwen_shape(device):
    """C1 widths (H=2048 -> 768, r=16) with the reference benchmark's skewed counts."""
    from art_amd.megatron.kernels.grouped_lora_hip import quack_grouped_lora
    e, d_in, d_out, r, m = 128, 2048, 768, 16, 8192
    gen = torch.Generator().manual_seed(1234)
    raw = torch.rand(e, generator=gen).pow(3.0)
    ids = torch.multinomial(raw / raw.sum(), m, replacement=True, generator=gen)
    counts = torch.bincount(ids, minlength=e)
    x = torch.randn(m, d_in, generator=gen).to(torch.bfloat16)
    a = (torch.randn(e, d_in, r, generator=gen) * 0.01).to(torch.bfloat16)
    b = (torch.randn(e, r, d_out, generator=gen) * 0.01).to(torch.bfloat16)
    g = torch.randn(m, d_out, generator=gen).to(torch.bfloat16)
    xr, ar, br = (v.float().requires_grad_() for v in (x, a, b))
    ref = OL.grouped_lora(xr, ar, br, counts.tolist(), 2.0)
    (ref * g.float()).sum().backward()
    xg, ag, bg = (v.to(device).requires_grad_() for v in (x, a, b))
    out = quack_grouped_lora(xg, ag, bg, counts.to(device), scale=2.0)
    (out.float() * g.to(device).float()).sum().backward()
    for got, want in ((out, ref), (xg.grad, xr.grad), (ag.grad, ar.grad), (bg.grad, br.grad)):
        assert rel(got, want) < 2e-2


def test_validation_errors(device):
    from art_amd.megatron.kernels.grouped_lora_hip import quack_grouped_lora
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=device)
    a = torch.zeros(2, 64, 9, dtype=torch.bfloat16, device=device)
    b = torch.zeros(2, 9, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="multiple of 8"):
        quack_grouped_lora(x, a, b, [2, 2])
    a = torch.zeros(2, 64, 8, dtype=torch.bfloat16, device=device)
    b = torch.zeros(2, 8, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="tokens_per_expert length"):
        quack_grouped_lora(x, a, b, [4])
    with pytest.raises(ValueError, match="Unsupported dtype"):
        quack_grouped_lora(x.float(), a, b, [2, 2])


def test_zero_rows_give_empty_outputs_and_zero_grads(device):
    """No rows (x.shape[0] == 0, every count 0): the operators return empty
    outputs and zero factor gradients, and the C-ABI products accept the null
    data pointer of an empty tensor."""
    from art_amd import ops
    from art_amd.megatron.kernels.grouped_lora_hip import quack_grouped_lora, quack_grouped_lora_dual
    e, h, out, r = 4, 64, 96, 8
    g = torch.Generator().manual_seed(11)
    x = torch.zeros(0, h, dtype=torch.bfloat16, device=device, requires_grad=True)
    a = (torch.randn(e, h, r, generator=g) * 0.1).to(torch.bfloat16).to(device).requires_grad_()
    b = (torch.randn(e, r, out, generator=g) * 0.1).to(torch.bfloat16).to(device).requires_grad_()
    counts = torch.zeros(e, dtype=torch.int64)
    y = quack_grouped_lora(x, a, b, counts, scale=2.0)
    assert y.shape == (0, out)
    y.backward(torch.zeros_like(y))   # the backward takes a row-major grad_out (reference contract)
    assert x.grad.shape == x.shape
    assert a.grad is not None and not a.grad.float().abs().any()
    assert b.grad is not None and not b.grad.float().abs().any()
    a2 = a.detach().clone().requires_grad_()
    b2 = b.detach().clone().requires_grad_()
    yd = quack_grouped_lora_dual(x, a, b, a2, b2, counts, scale_gate=2.0, scale_up=2.0)
    assert yd.shape == (0, 2 * out)
    # the C-ABI products themselves at M = 0
    seg = ops.segments_from_counts(counts, e, device)
    w = torch.randn(e, out, h, generator=g).to(torch.bfloat16).to(device)
    assert ops.grouped_gemm(x.detach(), w, seg, e, m=0).shape == (0, out)
    gw = ops.grouped_wgrad(x.detach(), torch.zeros(0, out, dtype=torch.bfloat16, device=device),
                           seg, e)
    assert gw.shape == (e, h, out) and not gw.abs().any()
