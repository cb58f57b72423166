"""Seeded synthetic workloads for the MoE-LoRA expert layer (the configs of the
benchmark specification, numbered C0..C4).

C0  tiny fp32-reference case: T=256, H=256, E=8, k=2, F=512, r=8, alpha=16
C1  Qwen3-30B-A3B expert layer: T=8192, H=2048, E=128, k=8, F=768, r=16
C2  C1 shapes with routing replay: Zipf(1.2) expert ids, Dirichlet(1) weights
C3  long context: T=32768, r=64, router LoRA rank 64 (A_r [H,64], B_r [64,E]),
    LoRA gradients accumulated in fp32
C4  wide layer: H=4096, F=1536, T=16384, r=32; base weights quantised to
    e4m3fn with per-output-channel fp32 scales (amax / 448), dequantised to
    bf16 inside the products (art_amd.quant)

Inputs follow the specification: x ~ N(0,1); base weights ~ N(0, 0.02);
LoRA A, B ~ N(0, 0.01) (B non-zero so both factors get gradients).  The
router weight is ~ N(0, 1/H) so that the router logits x W_r^T are ~ N(0,1)
(near-uniform load) as the C1 specification asks of the logits.  LoRA scale
is alpha / r with alpha = 32 (ART's LORA_ALPHA,
/root/reference/src/art/megatron/lora.py:40) unless the config says otherwise.

C2 replay targets: experts get Zipf ranks 1..E through a seeded permutation;
for each token, k distinct experts are drawn without replacement with
p(rank i) proportional to i^-1.2.  Because k distinct draws per token reach
every expert of a 128-way Zipf(1.2) within a few thousand tokens, the E/16
lowest-ranked experts get probability 0, which realises the configuration's
"some experts with 0 tokens".  The replayed gate weights are a Dirichlet(1)
sample per token, realised by setting the logits of the selected experts to
log(weight) (softmax over the selected logits then returns exactly those
weights).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class LayerConfig:
    name: str
    T: int
    H: int
    E: int
    k: int
    F: int
    r: int
    alpha: float = 32.0
    replay: bool = False
    note: str = ""
    router_r: int = 0       # router LoRA rank (0: none)
    fp8: bool = False       # frozen base weights stored as e4m3fn + per-row fp32 scales

    @property
    def scale(self) -> float:
        return self.alpha / self.r

    @property
    def M(self) -> int:
        return self.T * self.k

    def flops_fwd_bwd(self) -> dict:
        """Algorithmic FLOPs of one layer forward + backward (frozen base: dgrad only)."""
        m, h, f, r, e, t = self.M, self.H, self.F, self.r, self.E, self.T
        base_fc1 = 2 * m * h * 2 * f
        base_fc2 = 2 * m * f * h
        base = 2 * (base_fc1 + base_fc2)                       # fwd + dgrad
        lora = 3 * (2 * m * r * (h + f) * 2 + 2 * m * r * (f + h))  # gate, up, down; fwd + 2x bwd
        router = 4 * t * h * e                                 # fwd + dx
        rr = self.router_r
        router_lora = 6 * t * rr * (h + e)                     # fwd + dx + dA_r/dB_r
        return {"base": base, "lora": lora, "router": router, "router_lora": router_lora,
                "fc1_fwd": base_fc1, "fc2_fwd": base_fc2,
                "total": base + lora + router + router_lora}

    def dispatch_combine_bytes(self, b: int = 2) -> int:
        """HBM bytes of dispatch + combine, fwd + bwd, with materialised permutes."""
        return 4 * (self.T * self.H * b + self.M * self.H * b) + 4 * self.M * 4


CONFIGS = {
    "C0": LayerConfig("C0", T=256, H=256, E=8, k=2, F=512, r=8, alpha=16.0,
                      note="tiny; reference CPU case"),
    "C1": LayerConfig("C1", T=8192, H=2048, E=128, k=8, F=768, r=16,
                      note="Qwen3-30B-A3B expert layer"),
    "C2": LayerConfig("C2", T=8192, H=2048, E=128, k=8, F=768, r=16, replay=True,
                      note="C1 + Zipf(1.2) routing replay"),
    "C3": LayerConfig("C3", T=32768, H=2048, E=128, k=8, F=768, r=64, router_r=64,
                      note="long-context GRPO step, router LoRA, fp32 LoRA grad accumulation"),
    "C4": LayerConfig("C4", T=16384, H=4096, E=128, k=8, F=1536, r=32, fp8=True,
                      note="wide layer, fp8 e4m3fn base weights (per-output-channel scales)"),
}


def zipf_targets(t: int, e: int, k: int, s: float = 1.2, seed: int = 0,
                 n_empty: int | None = None) -> torch.Tensor:
    """k distinct experts per token, p(rank i) ~ i^-s without replacement (CPU, int64).

    The expert of rank i is perm[i-1] for a seeded permutation; the ``n_empty``
    (default E/16) lowest-ranked experts get probability 0.
    """
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(e, generator=g)
    n_empty = max(1, e // 16) if n_empty is None else n_empty
    if e - n_empty < k:
        raise ValueError("not enough experts with non-zero probability for k distinct draws")
    p_rank = torch.arange(1, e + 1, dtype=torch.float64).pow(-s)
    if n_empty:
        p_rank[e - n_empty:] = 0.0
    p = torch.zeros(e, dtype=torch.float64)
    p[perm] = p_rank
    p = (p / p.sum()).float()
    out = torch.empty((t, k), dtype=torch.int64)
    chunk = 4096
    for i in range(0, t, chunk):
        n = min(chunk, t - i)
        out[i:i + n] = torch.multinomial(p.expand(n, e), k, replacement=False, generator=g)
    return out


def dirichlet_weights(t: int, k: int, seed: int = 0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed + 1)
    gam = -torch.log(torch.rand((t, k), generator=g, dtype=torch.float64).clamp_min(1e-300))
    return (gam / gam.sum(1, keepdim=True)).float()


@dataclass
class LayerInputs:
    cfg: LayerConfig
    x: torch.Tensor
    w_r: torch.Tensor
    w1: torch.Tensor
    w2: torch.Tensor
    lora: dict            # a_g, b_g, a_u, b_u, a_d, b_d
    dy: torch.Tensor
    logits: torch.Tensor | None = None
    target: torch.Tensor | None = None
    extras: dict = field(default_factory=dict)


def make_inputs(cfg: LayerConfig, device="cpu", seed: int = 0, dtype=torch.bfloat16,
                T: int | None = None) -> LayerInputs:
    """Seeded inputs (generated on the CPU, then moved) for ``cfg`` (optionally fewer tokens)."""
    t = cfg.T if T is None else T
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape, std=1.0):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    e, h, f, r = cfg.E, cfg.H, cfg.F, cfg.r
    x = rnd(t, h)
    w_r = rnd(e, h, std=1.0 / math.sqrt(h))
    w1 = rnd(e, 2 * f, h, std=0.02)
    w2 = rnd(e, h, f, std=0.02)
    lora = {
        "a_g": rnd(e, h, r, std=0.01), "b_g": rnd(e, r, f, std=0.01),
        "a_u": rnd(e, h, r, std=0.01), "b_u": rnd(e, r, f, std=0.01),
        "a_d": rnd(e, f, r, std=0.01), "b_d": rnd(e, r, h, std=0.01),
    }
    if cfg.router_r:
        lora["a_r"] = rnd(h, cfg.router_r, std=0.01)
        lora["b_r"] = rnd(cfg.router_r, e, std=0.01)
    dy = rnd(t, h)
    logits = target = None
    if cfg.replay:
        target = zipf_targets(t, e, cfg.k, seed=seed)
        wts = dirichlet_weights(t, cfg.k, seed=seed)
        logits = torch.randn(t, e, generator=g)
        logits.scatter_(1, target, torch.log(wts))
    mv = lambda v: None if v is None else v.to(device)
    return LayerInputs(cfg, mv(x), mv(w_r), mv(w1), mv(w2), {kk: mv(v) for kk, v in lora.items()},
                       mv(dy), mv(logits), mv(target))
