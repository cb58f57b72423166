"""The fused layer's forward + backward captured in a HIP graph.

No op of the path synchronises with the host or records a memset (scratch is
cleared by kernels, segment tables are built on the device), so a whole
training step of the layer can be captured once and replayed.  Every replay
must equal the eager step bit for bit; eager work and synchronisations run
between the replays, and the graph's inputs are rewritten in place between
them to check that the replay reads them afresh.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

NAMES = ("a_g", "b_g", "a_u", "b_u", "a_d", "b_d")


def _setup(cfg_name, device, seed=0):
    from art_amd.megatron.moe_layer import FrozenExperts
    from art_amd.workloads import CONFIGS, make_inputs
    cfg = CONFIGS[cfg_name]
    inp = make_inputs(cfg, "cpu", seed=seed)
    base = FrozenExperts.build(inp.w_r.to(device), inp.w1.to(device), inp.w2.to(device))
    lora = {n: inp.lora[n].to(device).requires_grad_() for n in NAMES}
    x = inp.x.to(device).requires_grad_()
    return cfg, inp, base, lora, x


@pytest.mark.parametrize("cfg_name,replay", [("C0", False), ("C0", True)])
def test_layer_step_graph_replays_match_eager(device, cfg_name, replay):
    from art_amd.megatron.moe_layer import moe_lora_layer
    cfg, inp, base, lora, x = _setup(cfg_name, device)
    print(f"graph capture {cfg_name} replay={replay}", flush=True)
    s = cfg.scale
    dy = inp.dy.to(device)
    logits = target = None
    if replay:   # replayed routes: logits and a fixed target instead of the router
        g = torch.Generator().manual_seed(5)
        logits = torch.randn(cfg.T, cfg.E, generator=g).to(device)
        target = torch.stack([torch.randperm(cfg.E, generator=g)[:cfg.k] for _ in range(cfg.T)])
        target = target.to(torch.int32).to(device)

    def step():
        y, idx, counts, status = moe_lora_layer(x, base, *(lora[n] for n in NAMES), k=cfg.k,
                                                scales=(s, s, s), logits=logits, target=target)
        y.backward(dy)
        return y, idx, counts, status

    def clear_grads():
        x.grad = None
        for v in lora.values():
            v.grad = None

    def snapshot(outs):
        y, idx, counts, status = outs
        return ([y.detach().clone(), idx.clone(), counts.clone(), status.clone(), x.grad.clone()] +
                [lora[n].grad.clone() for n in NAMES])

    clear_grads()
    eager = snapshot(step())
    # torch's capture rules: warm up on a side stream, then capture.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            clear_grads()
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    clear_grads()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_outs = step()
    torch.cuda.synchronize()

    x_saved = x.detach().clone()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = snapshot(static_outs)
        for i, (a, b) in enumerate(zip(got, eager)):
            assert torch.equal(a, b), f"replay {rep}: output {i} differs from the eager step"
        # eager work between replays, then a changed input: the next replay must
        # see it (and the original input again must give the eager result back)
        (torch.randn(512, 512, device=device) @ torch.randn(512, 512, device=device)).sum().item()
        with torch.no_grad():
            x.mul_(-1.0 if rep == 0 else 1.0)
        if rep == 0:
            graph.replay()
            torch.cuda.synchronize()
            assert not torch.equal(static_outs[0], eager[0]), "replay ignored the rewritten input"
            with torch.no_grad():
                x.copy_(x_saved)
