"""Pins the float oracle (oracle/layer.py).  CPU only, float64.

Checks that do not restate the oracle's formulas:
* torch.autograd.gradcheck (central finite differences) of grouped LoRA,
  dual LoRA, weighted SwiGLU and the whole layer, including the router path;
* dense equivalence: with every expert sharing one weight the grouped ops equal
  a single dense product (no segmentation involved);
* the layer with identical experts equals one dense SwiGLU MLP per token
  (the k renormalised weights of each token sum to one) -- pins permute,
  combine and weighting wiring;
* SwiGLU at g = 0 is 0 and its gate-gradient there is u*p/2 (silu'(0) = 1/2).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import layer as L

KATS = json.loads((Path(__file__).parent / "golden" / "routing_kats.json").read_text())
D = torch.float64


def _rand(*shape, scale=1.0, seed=None):
    g = torch.Generator().manual_seed(seed) if seed is not None else None
    return (torch.randn(*shape, generator=g, dtype=D) * scale)


def test_grouped_lora_gradcheck_zero_token_expert():
    kat = KATS["lora_cutover"]
    counts = [c // 8 for c in kat["counts"]]  # [4, 0, 2, 3]: same zero-token pattern, small
    torch.manual_seed(0)
    m = sum(counts)
    x = _rand(m, 6).requires_grad_()
    a = _rand(4, 6, 3).requires_grad_()
    b = _rand(4, 3, 5).requires_grad_()
    assert torch.autograd.gradcheck(lambda x, a, b: L.grouped_lora(x, a, b, counts, 2.0), (x, a, b))


def test_grouped_lora_dual_gradcheck():
    counts = [2, 3, 0]
    torch.manual_seed(1)
    x = _rand(5, 4).requires_grad_()
    ag, bg = _rand(3, 4, 2).requires_grad_(), _rand(3, 2, 3).requires_grad_()
    au, bu = _rand(3, 4, 1).requires_grad_(), _rand(3, 1, 3).requires_grad_()
    f = lambda x, ag, bg, au, bu: L.grouped_lora_dual(x, ag, bg, au, bu, counts, 2.0, 3.0)
    assert torch.autograd.gradcheck(f, (x, ag, bg, au, bu))


def test_grouped_ops_dense_equivalence():
    counts = [3, 0, 5, 1]
    x = _rand(9, 8, seed=2)
    a1, b1 = _rand(8, 4, seed=3), _rand(4, 6, seed=4)
    w = _rand(6, 8, seed=5)
    a = a1.expand(4, 8, 4)
    b = b1.expand(4, 4, 6)
    got = L.grouped_lora(x, a, b, counts, 0.5)
    assert torch.allclose(got, 0.5 * (x @ a1 @ b1), atol=1e-12)
    got = L.grouped_linear(x, w.expand(4, 6, 8), counts)
    assert torch.allclose(got, x @ w.t(), atol=1e-12)


def test_weighted_swiglu_gradcheck_and_zero_gate():
    y1 = _rand(7, 10, seed=6).requires_grad_()
    p = torch.rand(7, dtype=D).requires_grad_()
    assert torch.autograd.gradcheck(L.weighted_swiglu, (y1, p))
    y1z = y1.detach().clone()
    y1z[:, :5] = 0.0
    y1z.requires_grad_()
    h = L.weighted_swiglu(y1z, p.detach())
    assert torch.all(h == 0)
    h.sum().backward()
    expect = 0.5 * y1z.detach()[:, 5:] * p.detach()[:, None]
    assert torch.allclose(y1z.grad[:, :5], expect, atol=1e-12)


def _params(e, h, f, r, seed, w_r=True, scale=0.3):
    g = torch.Generator().manual_seed(seed)
    rnd = lambda *s: torch.randn(*s, generator=g, dtype=D) * scale
    return L.LayerParams(
        w_r=rnd(e, h) if w_r else None, w1=rnd(e, 2 * f, h), w2=rnd(e, h, f),
        a_g=rnd(e, h, r), b_g=rnd(e, r, f), a_u=rnd(e, h, r), b_u=rnd(e, r, f),
        a_d=rnd(e, f, r), b_d=rnd(e, r, h), scale_g=2.0, scale_u=2.0, scale_d=2.0)


def test_layer_identical_experts_equals_dense_mlp():
    e, h, f, r, t, k = 5, 8, 6, 2, 11, 3
    p = _params(e, h, f, r, seed=8)
    for name in ("w1", "w2", "a_g", "b_g", "a_u", "b_u", "a_d", "b_d"):
        v = getattr(p, name)
        setattr(p, name, v[:1].expand_as(v).clone())
    x = _rand(t, h, seed=9)
    y, aux = L.moe_lora_layer(x, p, k, dtype=D)
    # one dense SwiGLU MLP with LoRA, no routing at all
    w1 = p.w1[0] + torch.cat((p.scale_g * (p.a_g[0] @ p.b_g[0]).t(), p.scale_u * (p.a_u[0] @ p.b_u[0]).t()), 0)
    w2 = p.w2[0] + p.scale_d * (p.a_d[0] @ p.b_d[0]).t()
    z = x @ w1.t()
    dense = (torch.nn.functional.silu(z[:, :f]) * z[:, f:]) @ w2.t()
    assert torch.allclose(y, dense, atol=1e-10)
    assert aux["plan"]["counts"].sum() == t * k


def test_layer_gradcheck_router_and_lora():
    e, h, f, r, t, k = 4, 4, 3, 2, 5, 2
    p = _params(e, h, f, r, seed=10)
    x = _rand(t, h, seed=11).requires_grad_()
    leaves = [x]
    names = ["a_g", "b_g", "a_u", "b_u", "a_d", "b_d"]
    for n in names:
        v = getattr(p, n).clone().requires_grad_()
        setattr(p, n, v)
        leaves.append(v)

    def fn(x, *lora):
        for n, v in zip(names, lora):
            setattr(p, n, v)
        y, _ = L.moe_lora_layer(x, p, k, dtype=D)
        return y

    # Routing is piecewise constant in x; the default finite-difference step
    # (1e-6) does not cross a top-k boundary for these random inputs.
    assert torch.autograd.gradcheck(fn, tuple(leaves), eps=1e-6, atol=1e-6)


def test_layer_replay_target_overrides_topk():
    e, h, f, r, t, k = 6, 8, 4, 2, 4, 2
    p = _params(e, h, f, r, seed=12)
    x = _rand(t, h, seed=13)
    target = torch.tensor([[5, 0], [0, 5], [2, 3], [3, 2]])
    _, aux = L.moe_lora_layer(x, p, k, target=target, dtype=D)
    assert aux["idx"].tolist() == target.tolist()
    assert aux["plan"]["counts"].tolist() == [2, 0, 2, 2, 0, 2]
    sel = aux["logits"].gather(1, target)
    assert torch.allclose(aux["w"], torch.softmax(sel, -1))


def test_layer_zero_tokens():
    p = _params(3, 8, 4, 2, seed=14)
    y, aux = L.moe_lora_layer(torch.zeros(0, 8, dtype=D), p, 2, dtype=D)
    assert y.shape == (0, 8)
    assert aux["plan"]["counts"].tolist() == [0, 0, 0]


def test_router_lora_equals_merged_router_weight():
    """x W^T + s (x A) B == x (W + s (A B)^T)^T: pins operand order and scale."""
    t, h, e, rr = 7, 6, 5, 3
    x = _rand(t, h, seed=20)
    w = _rand(e, h, seed=21)
    a = _rand(h, rr, seed=22)
    b = _rand(rr, e, seed=23)
    got = L.router_logits(x, w, D, a_r=a, b_r=b, scale_r=0.75)
    merged = L.router_logits(x, w + 0.75 * (a @ b).t(), D)
    assert torch.allclose(got, merged, atol=1e-12)
    assert torch.allclose(L.router_logits(x, w, D, a_r=a, b_r=torch.zeros_like(b), scale_r=2.0),
                          L.router_logits(x, w, D), atol=0)


def test_layer_gradcheck_router_lora():
    e, h, f, r, t, k = 4, 4, 3, 2, 5, 2
    p = _params(e, h, f, r, seed=30)
    p.a_r = _rand(h, 3, seed=31).requires_grad_()
    p.b_r = _rand(3, e, seed=32).requires_grad_()
    p.scale_r = 0.5
    x = _rand(t, h, seed=33).requires_grad_()

    def fn(x, a_r, b_r):
        p.a_r, p.b_r = a_r, b_r
        y, _ = L.moe_lora_layer(x, p, k, dtype=D)
        return y

    assert torch.autograd.gradcheck(fn, (x, p.a_r, p.b_r), eps=1e-6, atol=1e-6)


def test_layer_fused_gate_up_equals_dual_with_shared_a():
    """One gate|up adapter (A shared, B over 2F columns) is the dual form with
    A_g = A_u = A, B_g = B[:, :, :F], B_u = B[:, :, F:] at one scale; a swapped
    or transposed half breaks the identity.  Gradients by finite differences."""
    e, h, f, r, t, k = 4, 6, 3, 2, 6, 2
    p = _params(e, h, f, r, seed=40)
    x = _rand(t, h, seed=41)
    a = _rand(e, h, r, seed=42)
    b = _rand(e, r, 2 * f, seed=43)
    p.a_g, p.a_u, p.b_g, p.b_u = a, a, b[:, :, :f], b[:, :, f:]
    p.scale_u = p.scale_g
    y_dual, _ = L.moe_lora_layer(x, p, k, dtype=D)
    p.a_u = p.b_u = None
    p.b_g = b
    y_fused, _ = L.moe_lora_layer(x, p, k, dtype=D)
    assert torch.allclose(y_fused, y_dual, atol=1e-12)
    p.b_g = torch.cat((b[:, :, f:], b[:, :, :f]), dim=2)   # halves swapped
    y_swapped, _ = L.moe_lora_layer(x, p, k, dtype=D)
    assert not torch.allclose(y_swapped, y_dual, atol=1e-6)

    xl = x.clone().requires_grad_()
    al = a.clone().requires_grad_()
    bl = b.clone().requires_grad_()

    def fn(x, a, b):
        p.a_g, p.b_g = a, b
        y, _ = L.moe_lora_layer(x, p, k, dtype=D)
        return y

    assert torch.autograd.gradcheck(fn, (xl, al, bl), eps=1e-6, atol=1e-6)
