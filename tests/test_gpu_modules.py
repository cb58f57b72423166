"""Module-level mirrors on the GPU: megatron-signature permute / unpermute /
weighted_bias_swiglu_impl, the LoRA module and the expert MLP wrappers.

Bars: permutation order and sorted_indices bit-exact against megatron's
mask construction ``arange(T).expand(E, T).masked_select(routing_map.T)``;
permuted rows bit-exact; combine sums within one bf16 ulp of an fp32
index_add; SwiGLU and module outputs / gradients within 2e-2 of torch fp32;
the module path (permute -> GroupedMLP -> unpermute) equal to the fused layer
within 2e-2.
"""
import math

import numpy as np
import pytest
import torch

from oracle import layer as OL

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _routing(t, e, k, seed, device):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(t, e, generator=g)
    idx = torch.topk(logits, k, dim=1).indices
    rmap = torch.zeros(t, e, dtype=torch.bool).scatter_(1, idx, True)
    probs = torch.zeros(t, e).scatter_(1, idx, torch.softmax(logits.gather(1, idx), -1))
    return rmap.to(device), probs.to(device)


@pytest.mark.parametrize("t,e,k,h", [(300, 16, 4, 256), (1, 8, 2, 64), (64, 4, 4, 24)])
def test_permute_unpermute_megatron_order(device, t, e, k, h):
    from art_amd.megatron.moe_utils import permute, unpermute
    rmap, probs = _routing(t, e, k, t + e, device)
    x = torch.randn(t, h, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(device)
    out, pprobs, sorted_idx = permute(x, rmap, probs=probs, num_out_tokens=t * k)
    expect = torch.arange(t).expand(e, t).masked_select(rmap.cpu().t())
    assert torch.equal(sorted_idx.cpu(), expect)
    assert torch.equal(out.cpu(), x.cpu()[expect])
    assert torch.equal(pprobs.cpu(), probs.cpu().t().masked_select(rmap.cpu().t()))
    # token uids (int64 metadata) take the torch path with the same order
    uids, _, _ = permute(torch.arange(t, device=device).unsqueeze(-1), rmap, num_out_tokens=t * k)
    assert torch.equal(uids.cpu().view(-1), expect)
    y = unpermute(out, sorted_idx, x.shape)
    ref = torch.zeros(t, h).index_add(0, expect, out.cpu().float())
    torch.testing.assert_close(y.cpu().float(), ref, rtol=2 ** -8, atol=1e-6)
    yw = unpermute(out, sorted_idx, x.shape, probs=probs, routing_map=rmap)
    refw = torch.zeros(t, h).index_add(0, expect, out.cpu().float() * pprobs.cpu().unsqueeze(1))
    torch.testing.assert_close(yw.cpu().float(), refw, rtol=2 ** -7, atol=1e-5)


def test_permute_unpermute_gradients(device):
    from art_amd.megatron.moe_utils import permute, unpermute
    t, e, k, h = 200, 8, 2, 128
    rmap, probs = _routing(t, e, k, 5, device)
    x = torch.randn(t, h, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(device)
    x.requires_grad_()
    pr = probs.clone().requires_grad_()
    out, _, sidx = permute(x, rmap, num_out_tokens=t * k)
    y = unpermute(out, sidx, x.shape, probs=pr, routing_map=rmap)
    gy = torch.randn(t, h, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    y.backward(gy.to(device))
    # fp32 reference: y[t] = x[t] * sum_e probs[t, e] over the routed experts
    xr = x.detach().cpu().float().requires_grad_()
    prr = probs.cpu().clone().requires_grad_()
    yr = xr * (prr * rmap.cpu()).sum(1, keepdim=True)
    yr.backward(gy.float())
    assert rel(x.grad, xr.grad) < 2e-2
    assert rel(pr.grad * rmap, prr.grad * rmap.cpu()) < 2e-2


@pytest.mark.parametrize("t,e,k,h,cap_factor", [(300, 16, 4, 256, 1.0), (200, 8, 2, 128, 0.5),
                                                 (64, 4, 4, 24, 1.5)])
def test_permute_unpermute_capacity_layout(device, t, e, k, h, cap_factor):
    """drop_and_pad: rows follow the oracle's capacity layout (routed tokens
    ascending, the excess dropped, then non-routed padding ascending) bit for
    bit, probs are gathered at those (token, expert) pairs (0 on padding),
    unpermute sums within one bf16 ulp of an fp32 index_add, and gradients
    (rows and probs) match an fp32 torch restatement."""
    from art_amd.megatron.moe_utils import permute, unpermute
    from oracle import routing as R
    rmap, probs = _routing(t, e, k, t + 3 * e, device)
    n_out = int(t * k * cap_factor)
    cap = min(n_out // e, t)
    x = torch.randn(t, h, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(device)
    out, pprobs, sidx = permute(x, rmap, probs=probs, num_out_tokens=n_out, drop_and_pad=True)
    want = torch.from_numpy(R.capacity_layout(rmap.cpu().numpy(), cap))
    assert torch.equal(sidx.cpu(), want) and out.shape == (e * cap, h)
    assert torch.equal(out.cpu(), x.cpu()[want])
    expert = torch.arange(e * cap) // cap
    assert torch.equal(pprobs.cpu(), probs.cpu()[want, expert])
    uids, _, _ = permute(torch.arange(t, device=device).unsqueeze(-1), rmap, num_out_tokens=n_out,
                         drop_and_pad=True)
    assert torch.equal(uids.cpu().view(-1), want)
    y = unpermute(out, sidx, x.shape, routing_map=rmap, drop_and_pad=True)
    ref = torch.zeros(t, h).index_add(0, want, out.cpu().float())
    torch.testing.assert_close(y.cpu().float(), ref, rtol=2 ** -8, atol=1e-6)
    # weighted, with gradients
    xg = x.clone().requires_grad_()
    pg = probs.clone().requires_grad_()
    o2, _, s2 = permute(xg, rmap, num_out_tokens=n_out, drop_and_pad=True)
    yw = unpermute(o2, s2, x.shape, probs=pg, routing_map=rmap, drop_and_pad=True)
    refw = torch.zeros(t, h).index_add(0, want, out.cpu().float() *
                                       probs.cpu()[want, expert].unsqueeze(1))
    torch.testing.assert_close(yw.detach().cpu().float(), refw, rtol=2 ** -7, atol=1e-5)
    gy = torch.randn(t, h, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    yw.backward(gy.to(device))
    xr = x.detach().cpu().float().requires_grad_()
    prr = probs.cpu().clone().requires_grad_()
    yr = torch.zeros(t, h).index_add(0, want, xr[want] * prr[want, expert].unsqueeze(1))
    yr.backward(gy.float())
    assert rel(xg.grad, xr.grad) < 2e-2
    assert rel(pg.grad, prr.grad) < 2e-2
    with pytest.raises(ValueError, match="pad_offsets"):
        unpermute(out, sidx, x.shape, routing_map=rmap, drop_and_pad=True,
                  pad_offsets=torch.zeros(e, dtype=torch.int64, device=device))


def test_weighted_bias_swiglu_impl(device):
    from art_amd.megatron.moe_utils import weighted_bias_swiglu_impl
    m, f = 1000, 384
    g = torch.Generator().manual_seed(7)
    y1 = torch.randn(m, 2 * f, generator=g).to(torch.bfloat16)
    w = torch.rand(m, 1, generator=g)
    a, b = y1.to(device).requires_grad_(), w.to(device).requires_grad_()
    h = weighted_bias_swiglu_impl(a, None, b)
    dh = torch.randn(m, f, generator=g).to(torch.bfloat16)
    h.backward(dh.to(device))
    ar, br = y1.float().requires_grad_(), w.clone().requires_grad_()
    gg, uu = ar.chunk(2, -1)
    hr = torch.nn.functional.silu(gg) * uu * br
    hr.backward(dh.float())
    assert rel(h.detach(), hr.detach()) < 1e-2
    assert rel(a.grad, ar.grad) < 1e-2 and rel(b.grad, br.grad) < 1e-3
    empty = torch.zeros(0, 2 * f, device=device, dtype=torch.bfloat16, requires_grad=True)
    z = weighted_bias_swiglu_impl(empty, None, torch.zeros(0, 1, device=device))
    assert z.shape == (0, f) and z.requires_grad
    with pytest.raises(ValueError, match="bias"):
        weighted_bias_swiglu_impl(a, torch.zeros(2 * f, device=device), b)


def test_lora_module_init_forward_and_export(device):
    from art_amd.megatron.lora import LoRA
    e, din, dout, r = 4, 256, 192, 8
    torch.manual_seed(0)
    lora = LoRA("base.layers.0.mlp.experts.{expert}.up_proj", din, dout, r, 16, torch.bfloat16,
                device, num_local_experts=e)
    assert lora.A_T.shape == (e, din, r) and lora.B_T.shape == (e, r, dout) and lora.scale == 2.0
    bound = 1 / math.sqrt(din)  # kaiming_uniform(a=sqrt(5)) on [r, in]
    assert lora.A_T.abs().max().item() <= bound * 1.01 and lora.A_T.abs().max().item() > bound * 0.8
    assert torch.count_nonzero(lora.B_T) == 0
    with torch.no_grad():
        lora.B_T.normal_(0, 0.05)
    counts = [40, 0, 25, 35]
    x = torch.randn(100, din, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    y = lora(x.to(device), tokens_per_expert=counts)
    ref = OL.grouped_lora(x.float(), lora.A_T.detach().cpu().float(),
                          lora.B_T.detach().cpu().float(), counts, lora.scale)
    assert rel(y, ref) < 2e-2
    assert lora(x[:0].to(device), tokens_per_expert=[0, 0, 0, 0]).shape == (0, dout)
    sd = lora.sharded_lora_state_dict()
    assert set(sd) == {f"base.layers.0.mlp.experts.{i}.up_proj.lora_{ab}.weight"
                       for i in range(e) for ab in "AB"}
    assert sd["base.layers.0.mlp.experts.2.up_proj.lora_A.weight"].shape == (r, din)
    other = LoRA("base.layers.0.mlp.experts.{expert}.up_proj", din, dout, r, 16, torch.bfloat16,
                 device, num_local_experts=e)
    other.load_lora_state_dict(sd)
    assert torch.equal(other.A_T, lora.A_T) and torch.equal(other.B_T, lora.B_T)
    single = LoRA("q_proj", din, dout, r, 16, torch.bfloat16, device)
    assert single.A_T.shape == (din, r)
    with pytest.raises(ValueError, match="num_local_experts > 1"):
        single(x.to(device), tokens_per_expert=[100])


@pytest.mark.parametrize("fp8", [False, True])
def test_module_path_equals_fused_layer(device, fp8):
    """permute -> GroupedMLP(FC1 LoRA, weighted SwiGLU, FC2 LoRA) -> unpermute
    reproduces the fused layer's output and LoRA gradients."""
    from art_amd.megatron.lora import (GroupedLinear, GroupedMLP, MLPExpertsLinearFC1LoRA,
                                       MLPExpertsLinearFC2LoRA)
    from art_amd.megatron.moe_layer import FrozenExperts, moe_lora_layer
    from art_amd.megatron.moe_utils import permute, unpermute
    from art_amd.quant import dequantize_fp8_rows, quantize_fp8_rows
    t, h, e, k, f, r = 512, 256, 8, 2, 128, 16
    print(f"module path fp8={fp8}", flush=True)
    g = torch.Generator().manual_seed(11)
    w1 = (torch.randn(e, 2 * f, h, generator=g) * 0.02).to(device)
    w2 = (torch.randn(e, h, f, generator=g) * 0.02).to(device)
    if fp8:
        q1, s1 = quantize_fp8_rows(w1)
        q2, s2 = quantize_fp8_rows(w2)
        fc1, fc2 = GroupedLinear(q1, s1), GroupedLinear(q2, s2)
        base = FrozenExperts.build_fp8(None, q1, s1, q2, s2)
    else:
        w1, w2 = w1.to(torch.bfloat16), w2.to(torch.bfloat16)
        fc1, fc2 = GroupedLinear(w1), GroupedLinear(w2)
        base = FrozenExperts.build(None, w1, w2)
    m1 = MLPExpertsLinearFC1LoRA("experts", fc1, r, 32, e)
    m2 = MLPExpertsLinearFC2LoRA("experts", fc2, r, 32, e)
    with torch.no_grad():
        for p in (m1.gate_lora.B_T, m1.up_lora.B_T, m2.lora.B_T):
            p.normal_(0, 0.02)
    mlp = GroupedMLP(m1, m2)
    logits = torch.randn(t, e, generator=g).to(device)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16).to(device)
    dy = torch.randn(t, h, generator=g).to(torch.bfloat16).to(device)
    # module path (megatron order of operations)
    from art_amd import ops
    idx, w = ops.router_topk(logits, k)
    rmap = torch.zeros(t, e, dtype=torch.bool, device=device).scatter_(1, idx.long(), True)
    probs = torch.zeros(t, e, device=device).scatter_(1, idx.long(), w)
    xm = x.clone().requires_grad_()
    perm, pprobs, sidx = permute(xm, rmap, probs=probs, num_out_tokens=t * k)
    counts = rmap.sum(0).cpu().tolist()
    out, _ = mlp(perm, counts, pprobs)
    y_mod = unpermute(out, sidx, x.shape)
    y_mod.backward(dy)
    grads_mod = [p.grad.clone() for p in (m1.gate_lora.A_T, m1.gate_lora.B_T, m1.up_lora.A_T,
                                          m1.up_lora.B_T, m2.lora.A_T, m2.lora.B_T)]
    # fused layer, same routing and weights
    leaves = [p.detach().clone().requires_grad_() for p in (
        m1.gate_lora.A_T, m1.gate_lora.B_T, m1.up_lora.A_T, m1.up_lora.B_T, m2.lora.A_T, m2.lora.B_T)]
    xf = x.clone().requires_grad_()
    s = m1.gate_lora.scale
    y_f, _, _, _ = moe_lora_layer(xf, base, *leaves, k=k, scales=(s, s, s), logits=logits)
    y_f.backward(dy)
    assert rel(y_mod.detach(), y_f.detach()) < 2e-2
    assert rel(xm.grad, xf.grad) < 2e-2
    for a, b in zip(grads_mod, [l.grad for l in leaves]):
        assert rel(a, b) < 2e-2
