"""Dense LoRA linears: attention QKV + output projection, forward + backward.

Times ``art_amd.megatron.dense_lora`` on one GPU against the reference's own
composition of the same layer (base linear plus separate ``(x A) B * s``
products per adapter and the grouped-query concatenation,
/root/reference/src/art/megatron/lora.py:1344-1395, 1190-1201) run on torch's
bf16 GEMMs.  Shapes default to Qwen3-30B-A3B attention (hidden 2048, 32 heads,
4 KV groups, head dim 128, rank 16).  Synthetic bf16 data; one JSON line.

    python art-mlx_amd/bench_dense_lora.py [--tokens 8192] [--steps 20] [--warmup 3]
"""
from __future__ import annotations

import argparse
import json
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import torch  # noqa: E402

from art_amd.megatron.dense_lora import SelfAttentionLinearProjLoRA, SelfAttentionLinearQKVLoRA  # noqa: E402


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--hidden", type=int, default=2048)
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--groups", type=int, default=4)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--rank", type=int, default=16)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("bench_dense_lora needs a GPU")
    dev = "cuda"
    torch.manual_seed(0)
    t, h, heads, groups, d, r = (args.tokens, args.hidden, args.heads, args.groups,
                                 args.head_dim, args.rank)
    hpg = heads // groups
    qkv_out = groups * (hpg * d + 2 * d)
    wq = (torch.randn(qkv_out, h, device=dev) * 0.02).bfloat16()
    wo = (torch.randn(h, heads * d, device=dev) * 0.02).bfloat16()
    qkv = SelfAttentionLinearQKVLoRA("q", wq, r, 2 * r, num_attention_heads=heads,
                                     num_query_groups=groups, kv_channels=d)
    proj = SelfAttentionLinearProjLoRA("o", wo, r, 2 * r)
    loras = (qkv.q_proj_lora, qkv.k_proj_lora, qkv.v_proj_lora, proj.lora)
    with torch.no_grad():
        for lora in loras:
            lora.B_T.normal_(0, 0.02)
    x = torch.randn(t, h, device=dev).bfloat16().requires_grad_()
    xo = torch.randn(t, heads * d, device=dev).bfloat16().requires_grad_()
    dyq = torch.randn(t, qkv_out, device=dev).bfloat16()
    dyo = torch.randn(t, h, device=dev).bfloat16()

    def ours():
        y, _ = qkv(x)
        y.backward(dyq)
        y, _ = proj(xo)
        y.backward(dyo)

    leaves = [(l.A_T.detach().clone().requires_grad_(), l.B_T.detach().clone().requires_grad_(),
               l.scale) for l in loras]

    def composition():
        (aq, bq, s), (ak, bk, _), (av, bv, _), (ao, bo, so) = leaves
        q = ((x @ aq) @ bq) * s
        k = ((x @ ak) @ bk) * s
        v = ((x @ av) @ bv) * s
        ad = torch.cat([q.view(t, groups, hpg * d), k.view(t, groups, d),
                        v.view(t, groups, d)], -1).view(t, -1)
        (x @ wq.T + ad).backward(dyq)
        (xo @ wo.T + ((xo @ ao) @ bo) * so).backward(dyo)

    def timed(fn) -> float:
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps

    ms = timed(ours)
    ms_ref = timed(composition)
    # frozen base: forward and input gradient of both products
    base_flop = 2 * 2 * t * (qkv_out * h + h * heads * d)
    print(json.dumps({
        "workload": "attention QKV + O dense LoRA fwd+bwd", "tokens": t, "hidden": h,
        "heads": heads, "kv_groups": groups, "head_dim": d, "rank": r,
        "ms_per_step": round(ms, 4), "composition_ms_per_step": round(ms_ref, 4),
        "speedup": round(ms_ref / ms, 3), "tokens_per_s": round(t / ms * 1e3),
        "base_tflops": round(base_flop / ms / 1e9, 1), "data": "synthetic"}), flush=True)


if __name__ == "__main__":
    main()
