"""Routing-replay bundle, builder and controller (host logic, CPU).

Scenarios and known answers restate the reference's unit tests
(/root/reference/tests/unit/test_moe_routing_replay.py:40-524 and
tests/unit/test_moe_routing_real_path.py:329-352); the synthetic rows are
pinned by Python's stdlib ``random`` through the committed golden fixture.
"""
import json
import random
from pathlib import Path

import pytest
import torch
from torch import nn

from art_amd.megatron import routing_replay as RR

KEY = "chunk_00.layer_0000.mlp.router"
KATS = json.loads((Path(__file__).parent / "golden" / "routing_kats.json").read_text())
TOPO = RR.ParallelTopology(tp=1, ep=1, etp=1, dp=1, sp=False, cp=1, pp=1, vpp=1)


def route(rows, *, sample_index=None, micro_slot=None, num_experts=3):
    idx = torch.tensor(rows, dtype=torch.int32)
    return RR.RouterCallRoute(expert_indices=idx, expert_mask=torch.ones_like(idx, dtype=torch.bool),
                              num_experts=num_experts, sample_index=sample_index,
                              micro_slot=micro_slot)


def bundle_of(calls, n_uids):
    return RR.MoeRoutingReplayBundle(
        topology=TOPO, num_steps=1, max_topk=2, router_keys=[KEY],
        steps={0: RR.StepRoutes(routers={KEY: RR.StepRouterRoutes(calls=calls)},
                                global_token_uids=torch.arange(n_uids, dtype=torch.int64))})


def single_bundle():
    r = route([[0, 2], [1, 0], [2, 1], [1, 0]], sample_index=0)
    return bundle_of({0: r}, 4), r


def sampled_bundle():
    return bundle_of({0: route([[0, 2], [1, 0]], sample_index=0),
                      1: route([[2, 1], [0, 1]], sample_index=1)}, 2)


class Replay:
    """Records every target it is given; replays the last one (the megatron
    RouterReplay contract the controller drives)."""

    def __init__(self):
        self.target = None
        self.action = None
        self.seen = []

    def set_target_indices(self, t):
        self.target = t
        self.seen.append(t.detach().cpu().clone())

    def set_router_replay_action(self, action):
        self.action = action


class Router(nn.Module):
    def __init__(self, topk=2, replay="default"):
        super().__init__()
        self.topk = topk
        self.router_replay = Replay() if replay == "default" else replay
        self.config = type("Cfg", (), {"sequence_parallel": False, "context_parallel_size": 1,
                                       "moe_router_fusion": False})()

    def routing(self, logits):
        scores = torch.softmax(logits, dim=-1)
        if self.router_replay is not None and self.router_replay.target is not None:
            idx = self.router_replay.target.long()
        else:
            idx = torch.topk(scores, self.topk, dim=1).indices
        routing_map = torch.zeros_like(scores, dtype=torch.bool)
        routing_map[torch.arange(scores.shape[0]).unsqueeze(1), idx] = True
        return scores, routing_map


class Chunk(nn.Module):
    """module path decoder.layers.0.mlp.router"""

    def __init__(self, router=None):
        super().__init__()
        mlp = nn.Module()
        mlp.router = router if router is not None else Router()
        layer = nn.Module()
        layer.mlp = mlp
        self.decoder = nn.Module()
        self.decoder.layers = nn.ModuleList([layer])

    @property
    def router(self):
        return self.decoder.layers[0].mlp.router


def expected_map(rows, e=3):
    m = torch.zeros((len(rows), e), dtype=torch.bool)
    for t, r in enumerate(rows):
        m[t, r] = True
    return m


def controller(bundle, chunk):
    c = RR.MoeRoutingReplayController(bundle=bundle, strict=True, device="cpu")
    c.install_router_patches([chunk])
    return c


# ------------------------------------------------------------------ names
def test_router_keys_from_compiled_module_names():
    assert RR.build_router_key_from_module_name(
        chunk_index=0, module_name="module.decoder.layers.0._orig_mod.mlp.router") == KEY
    assert RR.build_router_key_from_module_name(
        chunk_index=3, module_name="module.decoder.layers.12.mlp._orig_mod.router"
    ) == "chunk_03.layer_0012.mlp.router"
    assert RR.build_router_key_from_trace_name("chunk1.decoder.layers.7.mlp.router") == \
        "chunk_01.layer_0007.mlp.router"
    with pytest.raises(RuntimeError, match="Unable to derive router key"):
        RR.build_router_key_from_module_name(chunk_index=0, module_name="decoder.layers.0.mlp")


def test_local_token_indexer_sequence_parallel():
    class PS(RR.SingleProcessParallelState):
        def get_tensor_model_parallel_world_size(self):
            return 2

        def get_tensor_model_parallel_rank(self):
            return 1
    ix = RR.TopologyAwareLocalTokenIndexer(parallel_state_module=PS())
    uids = torch.arange(256, dtype=torch.int64)
    kw = dict(global_token_uids=uids, sequence_parallel=True, context_parallel_size=1)
    assert torch.equal(ix.build_local_token_uids(num_local_tokens=256, **kw), uids)
    assert torch.equal(ix.build_local_token_uids(num_local_tokens=128, **kw), torch.arange(128, 256))


# ------------------------------------------------------------------ bundle
def test_bundle_roundtrip_and_on_disk_format(tmp_path):
    b, r = single_bundle()
    b.steps[0].routers[KEY].calls[0].expert_probs = torch.rand(4, 2)
    b.to_dir(tmp_path)
    manifest = json.loads((tmp_path / "manifest.json").read_text())
    assert manifest["format_version"] == "moe_routing_replay_v2"
    assert manifest["steps"]["0"]["file"] == "step_000000.safetensors"
    assert manifest["steps"]["0"]["routers"][KEY] == {"0": {"num_experts": 3, "sample_index": 0}}
    assert manifest["topology"] == {"tp": 1, "ep": 1, "etp": 1, "dp": 1, "sp": False, "cp": 1,
                                    "pp": 1, "vpp": 1}
    from safetensors.torch import load_file
    t = load_file(str(tmp_path / "step_000000.safetensors"))
    assert sorted(t) == sorted(["global_token_uids", f"{KEY}/call_0/expert_indices",
                                f"{KEY}/call_0/expert_mask", f"{KEY}/call_0/expert_probs"])
    assert t[f"{KEY}/call_0/expert_indices"].dtype == torch.int32
    assert t[f"{KEY}/call_0/expert_mask"].dtype == torch.bool
    loaded = RR.MoeRoutingReplayBundle.from_dir(tmp_path)
    assert (loaded.num_steps, loaded.max_topk, loaded.router_keys) == (1, 2, [KEY])
    lr = loaded.steps[0].routers[KEY].calls[0]
    assert torch.equal(lr.expert_indices, r.expert_indices)
    assert torch.equal(lr.expert_mask, r.expert_mask)
    assert torch.equal(lr.expert_probs, b.steps[0].routers[KEY].calls[0].expert_probs)
    assert lr.sample_index == 0


def test_bundle_validation_errors():
    with pytest.raises(RuntimeError, match="outside"):
        route([[0, 3]])
    with pytest.raises(RuntimeError, match="unique per step"):
        RR.StepRoutes(routers={KEY: RR.StepRouterRoutes(calls={0: route([[0, 1], [1, 2]])})},
                      global_token_uids=torch.tensor([5, 5]))
    with pytest.raises(RuntimeError, match="must match step global_token_uids"):
        bundle_of({0: route([[0, 1]])}, 2)
    with pytest.raises(RuntimeError, match="steps must contain exactly"):
        RR.MoeRoutingReplayBundle(topology=TOPO, num_steps=2, max_topk=2, router_keys=[KEY],
                                  steps=single_bundle()[0].steps)
    with pytest.raises(RuntimeError, match="exceeds bundle max_topk"):
        RR.MoeRoutingReplayBundle(
            topology=TOPO, num_steps=1, max_topk=1, router_keys=[KEY],
            steps=single_bundle()[0].steps)


# ------------------------------------------------------------ synthetic rows
def test_synthetic_rows_match_golden_fixture():
    for case in KATS["synthetic_replay_rows"]:
        rows = RR.synthetic_replay_rows(row_positions=torch.tensor(case["positions"]),
                                        num_experts=case["num_experts"], topk=case["topk"],
                                        dtype=torch.int64, seed=case["seed"])
        assert rows.tolist() == case["rows"]
        # the fixture's seed is the builder's formula for (sample, layer)
        assert case["seed"] == (case["sample_index"] + 1) * 1_000_003 + \
            (case["layer_index"] + 1) * 97_003


# ------------------------------------------------------------------ builder
class _Replay:
    def __init__(self, expert_indices, token_mask, num_experts):
        self.expert_indices, self.token_mask, self.num_experts = expert_indices, token_mask, num_experts


def _packed(routes, seq_len, num_experts, valid_len):
    n, k = len(routes), len(routes[0])
    idx = torch.zeros((1, seq_len, 1, k), dtype=torch.int32)
    idx[0, :n, 0] = torch.tensor(routes, dtype=torch.int32)
    mask = torch.zeros((1, seq_len), dtype=torch.bool)
    mask[0, :n] = True
    gid = torch.full((1, seq_len), -1)
    gid[0, :valid_len] = 0
    return {"moe_routing_replay": _Replay(idx, mask, num_experts), "group_ids": gid,
            "parent_ids": gid.clone(), "logprobs": torch.zeros((1, seq_len))}


def test_builder_uses_packed_sequence_sample_calls():
    packed = _packed([[0, 1], [10, 11], [20, 21]], seq_len=4, num_experts=22, valid_len=3)
    b = RR.build_moe_routing_replay_bundle_from_packed_tensors(
        packed_tensors=packed, global_grad_accumulation_sequences=1, topology=TOPO)
    r = b.steps[0].routers[KEY].calls[0]
    assert r.sample_index == 0
    rows = r.expert_indices.tolist()
    assert rows[:3] == [[0, 1], [10, 11], [20, 21]]
    seed = 1 * 1_000_003 + 1 * 97_003
    assert rows[3] == random.Random(seed + 4 * 1_299_709).sample(range(22), 2)
    assert torch.equal(b.steps[0].global_token_uids, torch.arange(4))


def test_builder_fills_dummy_micro_slots_and_rejects_missing_scored_routes():
    packed = _packed([[0, 1], [2, 3]], seq_len=3, num_experts=8, valid_len=2)
    b = RR.build_moe_routing_replay_bundle_from_packed_tensors(
        packed_tensors=packed, global_grad_accumulation_sequences=2, topology=TOPO)
    dummy = b.steps[0].routers[KEY].calls[1]
    assert dummy.micro_slot == 1 and dummy.sample_index is None
    seed = 1 * 1_000_003 + 1 * 97_003 + 2 * 9_176
    assert dummy.expert_indices.tolist() == [
        random.Random(seed + (p + 1) * 1_299_709).sample(range(8), 2) for p in range(3)]
    # a missing route inside a group, before a scored token of that group
    packed = _packed([[0, 1]], seq_len=3, num_experts=8, valid_len=3)
    packed["parent_ids"][0, 1:] = 7
    with pytest.raises(RuntimeError, match="missing MoE routes outside terminal"):
        RR.build_moe_routing_replay_bundle_from_packed_tensors(
            packed_tensors=packed, global_grad_accumulation_sequences=1, topology=TOPO)


# --------------------------------------------------------------- controller
def test_controller_installs_bundle_target():
    b, r = single_bundle()
    chunk = Chunk()
    c = controller(b, chunk)
    c.set_step(step_index=0, sample_index=[0])
    c.begin_micro(0, 0)
    c.set_local_input_token_uids(torch.arange(4))
    _, m = chunk.router.routing(torch.randn(4, 3))
    assert torch.equal(m, expected_map(r.expert_indices.tolist()))
    assert torch.equal(chunk.router.router_replay.seen[-1], r.expert_indices.long())
    assert chunk.router.router_replay.action == RR.RouterReplayAction.REPLAY_FORWARD
    c.finalize_step()
    c.remove_router_patches()
    assert RR.active_routing_replay_controller() is None


def test_controller_maps_explicit_token_uids_to_rows():
    b, r = single_bundle()
    chunk = Chunk()
    c = controller(b, chunk)
    c.set_step(step_index=0, sample_index=[0])
    c.begin_micro(0, 0)
    c.set_local_input_token_uids(torch.tensor([3, 1]))
    assert chunk.router.router_replay.seen == []   # installed at routing time, not before
    _, m = chunk.router.routing(torch.randn(2, 3))
    want = r.expert_indices[[3, 1]]
    assert torch.equal(chunk.router.router_replay.seen[0], want.long())
    assert torch.equal(m, expected_map(want.tolist()))
    c.finalize_step()


def test_controller_switches_prestaged_layouts():
    b, r = single_bundle()
    chunk = Chunk()
    c = controller(b, chunk)
    c.set_step(step_index=0, sample_index=[0])
    c.begin_micro(0, 0)
    c.prepare_micro_targets({"attention": torch.tensor([0, 1]), "gdn": torch.tensor([3, 1])})
    _, m_att = chunk.router.routing(torch.randn(2, 3))
    c.set_active_token_uid_key("gdn")
    _, m_gdn = chunk.router.routing(torch.randn(2, 3))
    seen = chunk.router.router_replay.seen
    assert torch.equal(seen[0], r.expert_indices[[0, 1]].long())
    assert torch.equal(seen[1], r.expert_indices[[3, 1]].long())
    assert torch.equal(m_att, expected_map([[0, 2], [1, 0]]))
    assert torch.equal(m_gdn, expected_map([[1, 0], [1, 0]]))
    with pytest.raises(RuntimeError, match="was not staged"):
        c.set_active_token_uid_key("vision")
    c.finalize_step()


def test_controller_negative_uids_get_synthetic_rows():
    b, r = single_bundle()
    chunk = Chunk()
    c = controller(b, chunk)
    c.set_step(step_index=0, sample_index=[0])
    c.begin_micro(0, 0)
    c.set_local_input_token_uids(torch.tensor([2, -1, 0, -1]))
    chunk.router.routing(torch.randn(4, 3))
    t = chunk.router.router_replay.seen[0]
    seed = 1 * 1_000_003 + 1 * 97_003
    assert t[0].tolist() == r.expert_indices[2].tolist() and t[2].tolist() == [0, 2]
    for p in (1, 3):
        assert t[p].tolist() == random.Random(seed + (p + 1) * 1_299_709).sample(range(3), 2)
    with pytest.raises(RuntimeError, match="outside the active dense"):
        c.set_local_input_token_uids(torch.tensor([9]))
    c.remove_router_patches()


def test_controller_finalize_fails_on_unconsumed_calls():
    b, _ = single_bundle()
    c = controller(b, Chunk())
    c.set_step(step_index=0, sample_index=[0])
    with pytest.raises(RuntimeError, match="consumption mismatch"):
        c.finalize_step()
    c.remove_router_patches()


def test_controller_reuses_route_for_recompute():
    b = sampled_bundle()
    chunk = Chunk()
    c = controller(b, chunk)
    c.set_step(step_index=0, sample_index=[0, 1])
    c.begin_micro(0, 0)
    c.set_local_input_token_uids(torch.arange(2))
    _, m0 = chunk.router.routing(torch.randn(2, 3))
    _, m0r = chunk.router.routing(torch.randn(2, 3))   # activation recompute
    c.begin_micro(1, 1)
    c.set_local_input_token_uids(torch.arange(2))
    _, m1 = chunk.router.routing(torch.randn(2, 3))
    calls = b.steps[0].routers[KEY].calls
    seen = chunk.router.router_replay.seen
    assert len(seen) == 2
    assert torch.equal(seen[0], calls[0].expert_indices.long())
    assert torch.equal(seen[1], calls[1].expert_indices.long())
    assert torch.equal(m0, expected_map(calls[0].expert_indices.tolist()))
    assert torch.equal(m0r, m0)
    assert torch.equal(m1, expected_map(calls[1].expert_indices.tolist()))
    c.finalize_step()
    c.remove_router_patches()


def test_controller_recompute_reuse_can_be_disabled():
    b = sampled_bundle()
    chunk = Chunk()
    c = RR.MoeRoutingReplayController(bundle=b, strict=True, device="cpu",
                                      allow_recompute_reuse=False)
    c.install_router_patches([chunk])
    c.set_step(step_index=0, sample_index=[0, 1])
    c.begin_micro(0, 0)
    c.set_local_input_token_uids(torch.arange(2))
    chunk.router.routing(torch.randn(2, 3))
    with pytest.raises(RuntimeError, match="recompute reuse is disabled"):
        chunk.router.routing(torch.randn(2, 3))
    c.remove_router_patches()


def test_controller_rejects_several_calls_per_micro():
    b = bundle_of({0: route([[0, 2]], sample_index=0), 1: route([[1, 0]], sample_index=0),
                   2: route([[2, 1]], sample_index=1)}, 1)
    chunk = Chunk()
    c = controller(b, chunk)
    c.set_step(step_index=0, sample_index=[0, 1])
    with pytest.raises(RuntimeError, match="exactly one router call"):
        c.begin_micro(0, 0)
    assert chunk.router.router_replay.seen == []
    c.remove_router_patches()


def test_controller_install_checks():
    b, _ = single_bundle()
    c = RR.MoeRoutingReplayController(bundle=b, strict=True, device="cpu")
    with pytest.raises(RuntimeError, match="moe_enable_routing_replay=True"):
        c.install_router_patches([Chunk(router=Router(replay=None))])
    fused = Router()
    fused.config.moe_router_fusion = True
    with pytest.raises(RuntimeError, match="moe_router_fusion=False"):
        RR.MoeRoutingReplayController(bundle=b, strict=True, device="cpu").install_router_patches(
            [Chunk(router=fused)])


def test_controller_rejects_masked_slots_and_topk_mismatch():
    b, r = single_bundle()
    r.expert_mask[0, 1] = False
    c = controller(b, Chunk())
    with pytest.raises(RuntimeError, match="masked slots are unsupported"):
        c.set_step(step_index=0, sample_index=[0])
    c.remove_router_patches()
    b, _ = single_bundle()
    c = controller(b, Chunk(router=Router(topk=1)))
    with pytest.raises(RuntimeError, match="topk does not match"):
        c.set_step(step_index=0, sample_index=[0])
    c.remove_router_patches()


def test_controller_legacy_call_order_without_micro_metadata():
    """Calls without sample metadata are taken in contiguous blocks per sample."""
    calls = {i: route([[i % 3, (i + 1) % 3]] * 2) for i in range(4)}
    b = bundle_of(calls, 2)
    c = controller(b, Chunk())
    c.set_step(step_index=0, sample_index=[1], global_grad_accumulation_sequences=2)
    assert c.call_plan(KEY) == [2, 3]
    c.set_step(step_index=0, sample_index=[0, 1], global_grad_accumulation_sequences=2)
    assert c.call_plan(KEY) == [0, 1, 2, 3]
    with pytest.raises(RuntimeError, match="not divisible"):
        c.set_step(step_index=0, sample_index=[0], global_grad_accumulation_sequences=3)
    with pytest.raises(RuntimeError, match="lacks sample metadata"):
        c.set_step(step_index=0, sample_index=None)
    c.remove_router_patches()


def test_device_replay_target_wrapper_and_cpu_fallback():
    """DeviceReplayTarget reads table[rows]; on a CPU device the controller's
    device path falls back to host targets (the device path needs a GPU)."""
    table = torch.tensor([[1, 2], [3, 0], [2, 1]], dtype=torch.int32)
    rows = torch.tensor([2, 0, 0, 1], dtype=torch.int32)
    d = RR.DeviceReplayTarget(table, rows)
    assert d.shape == (4, 2)
    assert torch.equal(d.materialize(), torch.tensor([[2, 1], [1, 2], [1, 2], [3, 0]]))
    scores = torch.arange(16, dtype=torch.float32).reshape(4, 4)
    rr = RR.RouterReplay()
    rr.set_target_indices(d)
    rr.set_router_replay_action(RR.RouterReplayAction.REPLAY_FORWARD)
    vals, ids = rr.get_replay_topk(scores, 2)
    assert torch.equal(ids, d.materialize()) and torch.equal(vals, scores.gather(1, ids))
    with pytest.raises(RuntimeError, match="table"):
        RR.DeviceReplayTarget(table, rows.view(2, 2))
