"""fp8 e4m3fn weights (W8A16): the products dequantise each weight to
bf16(q * scale) inside the kernel, so with the same tile schedule they must be
bit-identical to the bf16 kernels run on the dequantised weights; the layer
with fp8 weights then matches the CPU oracle on the dequantised weights to
the bf16 bar (2e-2).
"""
import numpy as np
import pytest
import torch

from oracle import layer as OL

pytestmark = pytest.mark.gpu


def _ops():
    from art_amd import ops
    return ops


def _counts(e, m, seed):
    rng = np.random.default_rng(seed)
    p = rng.random(e) ** 2
    p[rng.choice(e, size=max(1, e // 4), replace=False)] = 0
    return np.bincount(rng.choice(e, size=m, p=p / p.sum()), minlength=e).tolist()


@pytest.fixture(autouse=True)
def _default_tiles(monkeypatch):
    monkeypatch.delenv("ART_MOE_GEMM_TILE", raising=False)


def test_quantize_roundtrip_matches_torch_e4m3fn(device):
    from art_amd.quant import dequantize_fp8_rows, quantize_fp8_rows
    w = torch.randn(3, 40, 128, generator=torch.Generator().manual_seed(1)) * 0.02
    q, s = quantize_fp8_rows(w.to(device))
    qc, sc = quantize_fp8_rows(w)
    torch.testing.assert_close(s.cpu(), sc, rtol=1e-6, atol=0)   # torch's GPU division may differ by an ulp
    assert (q.cpu().view(torch.uint8) != qc.view(torch.uint8)).float().mean().item() < 1e-3
    d = dequantize_fp8_rows(qc, sc).float()
    assert ((d - w).norm() / w.norm()).item() < 0.04          # e4m3: 3 mantissa bits
    assert torch.equal(qc.float().abs().amax(-1), torch.full((3, 40), 448.0))


@pytest.mark.parametrize("kt", [0, 32])
def test_fp8_products_bit_identical_to_bf16_on_dequantised_weights(device, kt):
    from art_amd.quant import dequantize_fp8_rows, quantize_fp8_rows, transpose_fp8
    ops = _ops()
    e, m, h, f = 8, 3000, 512, 256
    print(f"fp8 products kt={kt}", flush=True)
    g = torch.Generator().manual_seed(kt + 3)
    counts = _counts(e, m, seed=4)
    seg = ops.segments_from_counts(counts, e, device)
    w1 = (torch.randn(e, 2 * f, h, generator=g) * 0.02).to(device)
    w2 = (torch.randn(e, h, f, generator=g) * 0.02).to(device)
    q1, s1 = quantize_fp8_rows(w1)
    q2, s2 = quantize_fp8_rows(w2)
    d1, d2 = dequantize_fp8_rows(q1, s1), dequantize_fp8_rows(q2, s2)
    q1t, q2t = transpose_fp8(q1), transpose_fp8(q2)
    d1t, d2t = d1.transpose(1, 2).contiguous(), d2.transpose(1, 2).contiguous()
    t_src = 900
    x = torch.randn(t_src, h, generator=g).to(torch.bfloat16).to(device)
    rows = torch.randint(0, t_src, (m,), generator=g, dtype=torch.int32).to(device)
    prob = torch.rand(m, generator=g).to(device)
    lora = {}
    if kt:
        lora = dict(t1=torch.randn(m, kt, generator=g).to(torch.bfloat16).to(device),
                    l1=(torch.randn(e, 2 * f, kt, generator=g) * 0.1).to(torch.bfloat16).to(device),
                    l2=(torch.randn(e, h, kt, generator=g) * 0.1).to(torch.bfloat16).to(device),
                    l3=(torch.randn(e, f, kt, generator=g) * 0.1).to(torch.bfloat16).to(device),
                    l4=(torch.randn(e, h, kt, generator=g) * 0.1).to(torch.bfloat16).to(device))
    # FC1 + SwiGLU (row scales)
    k1 = dict(tl=lora["t1"], l1=lora["l1"]) if kt else {}
    y1a, ha = ops.fc1_swiglu(x, q1, seg, e, prob, m=m, a_rows=rows, w1_scale=s1, **k1)
    y1b, hb = ops.fc1_swiglu(x, d1, seg, e, prob, m=m, a_rows=rows, **k1)
    assert torch.equal(y1a, y1b) and torch.equal(ha, hb)
    # FC2 forward (row scales)
    k2 = dict(tl=lora["t1"], l=lora["l2"]) if kt else {}
    a = torch.randn(m, f, generator=g).to(torch.bfloat16).to(device)
    assert torch.equal(ops.grouped_gemm(a, q2, seg, e, b_scale=s2, **k2),
                       ops.grouped_gemm(a, d2, seg, e, **k2))
    # FC2 data gradient + SwiGLU backward (per-k scales of W2^T)
    k3 = dict(tl=lora["t1"], l2=lora["l3"]) if kt else {}
    dy = torch.randn(t_src, h, generator=g).to(torch.bfloat16).to(device)
    r1 = ops.fc2_dgrad_swiglu(dy, q2t, seg, e, y1b, prob, m=m, a_rows=rows, w2_scale=s2, **k3)
    r2 = ops.fc2_dgrad_swiglu(dy, d2t, seg, e, y1b, prob, m=m, a_rows=rows, **k3)
    assert torch.equal(r1[0], r2[0]) and torch.equal(r1[1], r2[1])
    # FC1 data gradient (per-k scales of W1^T)
    k4 = dict(tl=lora["t1"], l=lora["l4"]) if kt else {}
    assert torch.equal(ops.grouped_gemm(r2[0], q1t, seg, e, b_scale=s1, scale_per_k=True, **k4),
                       ops.grouped_gemm(r2[0], d1t, seg, e, **k4))
    torch.cuda.synchronize()


def test_fp8_argument_checks(device):
    from art_amd.quant import quantize_fp8_rows
    ops = _ops()
    seg = ops.segments_from_counts([4, 4], 2, device)
    a = torch.randn(8, 80, device=device).to(torch.bfloat16)
    q, s = quantize_fp8_rows(torch.randn(2, 32, 80, device=device))
    with pytest.raises(ValueError, match="multiple of 64"):
        ops.grouped_gemm(a, q, seg, 2, b_scale=s)
    with pytest.raises(ValueError, match="scales"):
        ops.grouped_gemm(a[:, :64].contiguous(), q[:, :, :64].contiguous(), seg, 2)


def test_layer_fp8_weights_c4_widths(device):
    """C4 widths (H=4096, F=1536, r=32) with 16 experts and 256 tokens: y, dx
    and LoRA gradients against the oracle on the dequantised weights."""
    import dataclasses
    from art_amd.megatron.moe_layer import FrozenExperts, moe_lora_layer
    from art_amd.quant import dequantize_fp8_rows, quantize_fp8_rows
    from art_amd.workloads import CONFIGS, make_inputs
    print("layer C4 fp8 widths E=16 T=256", flush=True)
    cfg = dataclasses.replace(CONFIGS["C4"], E=16)
    inp = make_inputs(cfg, "cpu", seed=0, T=256)
    q1, s1 = quantize_fp8_rows(inp.w1.to(device))
    q2, s2 = quantize_fp8_rows(inp.w2.to(device))
    base = FrozenExperts.build_fp8(inp.w_r.to(device), q1, s1, q2, s2)
    names = ("a_g", "b_g", "a_u", "b_u", "a_d", "b_d")
    lora = {n: inp.lora[n].to(device).requires_grad_() for n in names}
    x = inp.x.to(device).requires_grad_()
    s = cfg.scale
    y, idx, counts, _ = moe_lora_layer(x, base, *(lora[n] for n in names), k=cfg.k,
                                       scales=(s, s, s))
    y.backward(inp.dy.to(device))
    torch.cuda.synchronize()
    # oracle on the dequantised weights, replaying the GPU's selection
    w1d, w2d = dequantize_fp8_rows(q1, s1).cpu(), dequantize_fp8_rows(q2, s2).cpu()
    xo = inp.x.float().requires_grad_()
    leaves = {n: inp.lora[n].float().requires_grad_() for n in names}
    p = OL.LayerParams(w_r=inp.w_r, w1=w1d, w2=w2d, scale_g=s, scale_u=s, scale_d=s, **leaves)
    yo, _ = OL.moe_lora_layer(xo, p, cfg.k, target=idx.cpu().long())
    yo.backward(inp.dy.float())

    def rel(a, b):
        return ((a.double() - b.double()).norm() / b.double().norm()).item()
    errs = {"y": rel(y.detach().cpu(), yo.detach()), "dx": rel(x.grad.cpu(), xo.grad)}
    for n in names:
        errs["d" + n] = rel(lora[n].grad.cpu(), leaves[n].grad)
    print("  rel errs", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert all(v < 2e-2 for v in errs.values()), errs
