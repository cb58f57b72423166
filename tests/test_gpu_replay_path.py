"""Routing replay end to end on the GPU: a bundle written and read in the
reference's on-disk format, the controller staging per-micro targets to the
device, and the HIP router / fused layer consuming them.

Bar: replayed indices, counts and routing maps bit-exact against the bundle
rows of the micro's token uids; router weights and their logit gradients
against the CPU oracle (fp32, 1e-6).
"""
import numpy as np
import pytest
import torch

from oracle import routing as R

pytestmark = pytest.mark.gpu
KEY = "chunk_00.layer_0000.mlp.router"


class _Chunk(torch.nn.Module):
    def __init__(self, router):
        super().__init__()
        mlp = torch.nn.Module()
        mlp.router = router
        layer = torch.nn.Module()
        layer.mlp = mlp
        self.decoder = torch.nn.Module()
        self.decoder.layers = torch.nn.ModuleList([layer])


def _bundle(rows, num_experts, tmp_path):
    from art_amd.megatron import routing_replay as RR
    idx = torch.as_tensor(rows, dtype=torch.int32)
    call = RR.RouterCallRoute(expert_indices=idx, expert_mask=torch.ones_like(idx, dtype=torch.bool),
                              num_experts=num_experts, sample_index=0)
    b = RR.MoeRoutingReplayBundle(
        topology=RR.ParallelTopology(tp=1, ep=1), num_steps=1, max_topk=idx.shape[1],
        router_keys=[KEY],
        steps={0: RR.StepRoutes(routers={KEY: RR.StepRouterRoutes(calls={0: call})},
                                global_token_uids=torch.arange(idx.shape[0], dtype=torch.int64))})
    b.to_dir(tmp_path)
    return RR.MoeRoutingReplayBundle.from_dir(tmp_path)


@pytest.mark.parametrize("device_targets", [False, True])
def test_controller_targets_drive_hip_router_and_layer(device, tmp_path, device_targets):
    """Host path (host-gathered [T, k] target per router call) and device path
    (route table once per step + row map once per micro, replayed by the
    row-map kernel) give the same routing."""
    from art_amd import ops
    from art_amd.megatron import routing_replay as RR
    from art_amd.megatron.moe_layer import FrozenExperts, moe_lora_layer
    from art_amd.megatron.router import TopKRouter
    from art_amd.workloads import zipf_targets

    t, h, e, k, f, r = 2048, 256, 128, 8, 128, 16
    rows = zipf_targets(t, e, k, seed=3)          # Zipf(1.2) ids, some experts empty
    bundle = _bundle(rows, e, tmp_path)
    router = TopKRouter(h, e, k, moe_enable_routing_replay=True, device=device)
    ctl = RR.MoeRoutingReplayController(bundle=bundle, strict=True, device=device,
                                        device_targets=device_targets)
    ctl.install_router_patches([_Chunk(router)])
    ctl.set_step(step_index=0, sample_index=[0])
    ctl.begin_micro(0, 0)
    g = torch.Generator().manual_seed(5)
    uids = torch.randperm(t, generator=g)[:1500]   # the micro's tokens, out of order
    ctl.set_local_input_token_uids(uids)
    x = torch.randn(1500, h, generator=g).to(torch.bfloat16).to(device)
    logits = router.gating(x)
    probs, rmap = router.routing(logits)
    want = rows[uids]
    staged = router.router_replay.target_topk_idx
    assert isinstance(staged, RR.DeviceReplayTarget) == device_targets
    if device_targets:
        assert staged.shape == (1500, k) and staged.table.shape == (t, k)
        staged = staged.materialize()
    assert torch.equal(staged.cpu(), want)
    exp_map = torch.zeros((1500, e), dtype=torch.bool)
    exp_map[torch.arange(1500).unsqueeze(1), want] = True
    assert torch.equal(rmap.cpu(), exp_map)
    assert int(router.last_status.item()) == 0
    _, exp_w = R.replay(logits.detach().cpu().numpy(), want.numpy())
    np.testing.assert_allclose(probs.gather(1, want.to(device)).detach().cpu().numpy(), exp_w,
                               rtol=2e-6, atol=1e-7)
    # the fused layer consumes the same staged target
    target = router.router_replay.target_topk_idx
    wts = [torch.randn(e, 2 * f, h, generator=g) * 0.02, torch.randn(e, h, f, generator=g) * 0.02]
    base = FrozenExperts.build(router.weight, *(w.to(torch.bfloat16).to(device) for w in wts))
    lora = [(torch.randn(s, generator=g) * 0.01).to(torch.bfloat16).to(device)
            for s in [(e, h, r), (e, r, f), (e, h, r), (e, r, f), (e, f, r), (e, r, h)]]
    y, idx, counts, status = moe_lora_layer(x, base, *lora, k=k, scales=(2.0, 2.0, 2.0),
                                            target=target)
    assert torch.equal(idx.cpu().long(), want)
    assert counts.cpu().tolist() == torch.bincount(want.reshape(-1), minlength=e).tolist()
    assert int(status.item()) == 0
    ctl.finalize_step()
    ctl.remove_router_patches()


def test_topk_router_module_matches_oracle(device):
    from art_amd.megatron.router import TopKRouter
    t, h, e, k = 1000, 512, 64, 6
    router = TopKRouter(h, e, k, device=device)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16).to(device)
    logits = router.gating(x).detach().requires_grad_()
    exp_logits = x.float().cpu() @ router.weight.float().cpu().T
    torch.testing.assert_close(logits.detach().cpu(), exp_logits, rtol=1e-5, atol=1e-5)
    probs, rmap = router.routing(logits)
    exp_idx, exp_w = R.topk_softmax(logits.detach().cpu().numpy(), k)
    idx = torch.from_numpy(exp_idx).long()
    exp_map = torch.zeros((t, e), dtype=torch.bool)
    exp_map[torch.arange(t).unsqueeze(1), idx] = True
    assert torch.equal(rmap.cpu(), exp_map)
    np.testing.assert_allclose(probs.detach().cpu().gather(1, idx).numpy(), exp_w, rtol=2e-6,
                               atol=1e-7)
    # softmax-over-selected backward vs torch autograd on the CPU
    gout = torch.randn(t, e, generator=g)
    (probs * gout.to(device)).sum().backward()
    lc = logits.detach().cpu().requires_grad_()
    sel = torch.softmax(lc.gather(1, idx), dim=1)
    (sel * gout.gather(1, idx)).sum().backward()
    torch.testing.assert_close(logits.grad.cpu(), lc.grad, rtol=1e-5, atol=1e-6)


def test_device_targets_with_uidless_tokens_equal_host_targets(device, tmp_path):
    """Tokens without a uid (negative) get synthetic rows; on the device path
    they come from the per-call side table the row map addresses with
    negative entries.  Two routers, two micros, two uid layouts: every
    installed target equals the host path's, and both replay identically."""
    from art_amd import ops
    from art_amd.megatron import routing_replay as RR
    from art_amd.megatron.router import TopKRouter

    t, h, e, k = 512, 64, 32, 4
    g = torch.Generator().manual_seed(7)
    keys = ["chunk_00.layer_0000.mlp.router", "chunk_00.layer_0001.mlp.router"]

    def call(sample):
        idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)]).to(torch.int32)
        return RR.RouterCallRoute(expert_indices=idx, expert_mask=torch.ones_like(idx, dtype=torch.bool),
                                  num_experts=e, sample_index=sample)
    steps = {0: RR.StepRoutes(routers={rk: RR.StepRouterRoutes(calls={0: call(0), 1: call(1)})
                                       for rk in keys},
                              global_token_uids=torch.arange(1000, 1000 + t, dtype=torch.int64))}
    bundle = RR.MoeRoutingReplayBundle(topology=RR.ParallelTopology(tp=1, ep=1), num_steps=1,
                                       max_topk=k, router_keys=keys, steps=steps)
    bundle.to_dir(tmp_path)
    bundle = RR.MoeRoutingReplayBundle.from_dir(tmp_path)

    class Two(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.decoder = torch.nn.Module()
            self.decoder.layers = torch.nn.ModuleList()
            for _ in keys:
                layer = torch.nn.Module()
                layer.mlp = torch.nn.Module()
                layer.mlp.router = TopKRouter(h, e, k, moe_enable_routing_replay=True, device=device)
                self.decoder.layers.append(layer)

    uid_sets = []
    for micro in range(2):
        a = 1000 + torch.randperm(t, generator=g)[:300]
        a[torch.randperm(300, generator=g)[:17]] = -1          # tokens without a uid
        b = a.flip(0).clone()
        uid_sets.append({"attention": a, "gdn": b})
    logits = [torch.randn(300, e, generator=g).to(device) for _ in range(2)]

    def run(device_targets):
        model = Two()
        ctl = RR.MoeRoutingReplayController(bundle=bundle, strict=True, device=device,
                                            device_targets=device_targets)
        ctl.install_router_patches([model])
        ctl.set_step(step_index=0, sample_index=[0, 1])
        out = []
        for micro in range(2):
            ctl.begin_micro(micro, micro)
            ctl.prepare_micro_targets(uid_sets[micro])
            for layout in ("attention", "gdn"):
                ctl.set_active_token_uid_key(layout)
                for layer in model.decoder.layers:
                    r = layer.mlp.router
                    probs, rmap = r.routing(logits[micro])
                    tgt = r.router_replay.target_topk_idx
                    assert isinstance(tgt, RR.DeviceReplayTarget) == device_targets
                    ids = tgt.materialize() if device_targets else tgt
                    out.append((ids.cpu(), probs.detach().cpu(), int(r.last_status.item())))
        ctl.finalize_step()
        ctl.remove_router_patches()
        return out

    host, dev = run(False), run(True)
    assert len(host) == len(dev) == 8
    for (hi, hp, hs), (di, dp, ds) in zip(host, dev):
        assert torch.equal(hi, di) and torch.equal(hp, dp) and hs == ds == 0
    # the synthetic rows follow the stdlib formula: seed (step+1)*1_000_003 + (call+1)*97_003
    import random
    a = uid_sets[0]["attention"]
    p = int(torch.nonzero(a < 0)[0])
    want = random.Random(1 * 1_000_003 + 1 * 97_003 + (p + 1) * 1_299_709).sample(range(e), k)
    assert host[0][0][p].tolist() == want


def test_aligned_vllm_routes_replay_bit_exact(device, tmp_path):
    """vLLM route capture end to end: routes aligned from two choices' vLLM
    metadata, packed with a shared prompt, built into a bundle, written, read
    back straight into device route tables, staged by the controller and
    replayed by the HIP router: every captured token replays its captured
    experts bit for bit, in both layers."""
    import math
    from art_amd.megatron import routing_replay as RR
    from art_amd.megatron.router import TopKRouter
    from art_amd.preprocessing import moe_routing as MR
    from art_amd.preprocessing.pack import TokenizedResult, packed_tensors_from_tokenized_results

    e, k, n_layers, h = 64, 4, 2, 64
    g = torch.Generator().manual_seed(21)

    def routes(n):
        return [[torch.randperm(e, generator=g)[:k].tolist() for _ in range(n_layers)]
                for _ in range(n)]

    class Choice:
        def __init__(self, meta):
            self.model_extra = {MR.ART_MOE_ROUTING_METADATA_KEY: meta}

    prompt = list(range(100, 120))
    shared = routes(len(prompt))
    results = []
    for j, completion in enumerate([[7, 8, 9, 10, 11], [7, 8, 12, 13]]):
        meta = {"prompt_token_ids": prompt, "completion_token_ids": completion,
                "prompt_routed_experts": shared, "completion_routed_experts": routes(len(completion))}
        ids = prompt + completion
        aligned, stats = MR.align_choice_routes_to_tokenized_result(
            token_ids=ids, choices=[Choice(meta)], choice_offsets=[len(prompt)],
            choice_token_lengths=[len(completion)])
        assert stats.routed_tokens == len(ids) and aligned[len(prompt)] == \
            meta["completion_routed_experts"][0]
        n, pl = len(ids), len(prompt)
        results.append(TokenizedResult(token_ids=ids, input_pos=list(range(n)),
                                       assistant_mask=[0] * pl + [1] * (n - pl),
                                       logprobs=[math.nan] * pl + [-1.0] * (n - pl),
                                       advantage=1.0 + j, prompt_id=5, prompt_length=pl,
                                       moe_routed_experts=aligned))
    packed = packed_tensors_from_tokenized_results(results, seq_len=64, pad_token_id=0,
                                                   truncate_long_results=False,
                                                   include_moe_routing=True)
    rr = packed["moe_routing_replay"]
    assert rr.pack_stats.prefix_tree_rows == len(prompt) - 1       # shared but the last
    assert rr.pack_stats.prefix_tree_conflict_slots == 0
    bundle = RR.build_moe_routing_replay_bundle_from_packed_tensors(
        packed_tensors=packed, global_grad_accumulation_sequences=1,
        topology=RR.ParallelTopology(tp=1, ep=1))
    bundle.to_dir(tmp_path)
    on_host = RR.MoeRoutingReplayBundle.from_dir(tmp_path)
    on_dev = RR.MoeRoutingReplayBundle.from_dir(tmp_path, device=device)
    keys = [f"chunk_00.layer_{i:04d}.mlp.router" for i in range(n_layers)]
    for rk in keys:
        a = on_host.steps[0].routers[rk].calls[0].expert_indices
        b = on_dev.steps[0].routers[rk].calls[0].expert_indices
        assert b.device.type == "cuda" and torch.equal(a, b.cpu())

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.decoder = torch.nn.Module()
            self.decoder.layers = torch.nn.ModuleList()
            for _ in keys:
                layer = torch.nn.Module()
                layer.mlp = torch.nn.Module()
                layer.mlp.router = TopKRouter(h, e, k, moe_enable_routing_replay=True,
                                              device=device)
                self.decoder.layers.append(layer)

    model = Model()
    ctl = RR.MoeRoutingReplayController(bundle=on_dev, strict=True, device=device,
                                        device_targets=True)
    ctl.install_router_patches([model])
    ctl.set_step(step_index=0, sample_index=[0])
    ctl.begin_micro(0, 0)
    seq = int(packed["tokens"].shape[1])
    ctl.set_local_input_token_uids(torch.arange(seq))
    captured = rr.token_mask[0]
    logits = torch.randn(seq, e, generator=g).to(device)
    for li, layer in enumerate(model.decoder.layers):
        r = layer.mlp.router
        probs, rmap = r.routing(logits)
        tgt = r.router_replay.target_topk_idx
        assert isinstance(tgt, RR.DeviceReplayTarget)
        got = tgt.materialize().cpu()
        want = rr.expert_indices[0, :, li, :].long()
        assert torch.equal(got[captured], want[captured])
        assert torch.equal(got, on_host.steps[0].routers[keys[li]].calls[0].expert_indices.long())
        exp_map = torch.zeros((seq, e), dtype=torch.bool)
        exp_map[torch.arange(seq).unsqueeze(1), got] = True
        assert torch.equal(rmap.cpu(), exp_map)
        assert int(r.last_status.item()) == 0
    ctl.finalize_step()
    ctl.remove_router_patches()
