"""GPU parity of the routing family: top-k, replay, dispatch plan, permute, combine.

Bar: bit-exact indices / counts / offsets / destination rows / row->token maps
against the CPU oracle (oracle/routing.py), at the full C1/C2 sizes and on the
reference's own KAT routes; weights within 1e-6 of the oracle's softmax.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import routing as R

pytestmark = pytest.mark.gpu
KATS = json.loads((Path(__file__).parent / "golden" / "routing_kats.json").read_text())


def _ops():
    from art_amd import ops
    return ops


def _seg_expect(counts, e):
    counts = np.asarray(counts, dtype=np.int64)
    rows = [np.concatenate([[0], np.cumsum(counts)])]
    for bm in (64, 128, 192, 256, 2048):
        rows.append(np.concatenate([[0], np.cumsum((counts + bm - 1) // bm)]))
    return np.concatenate(rows)


def _check_plan(plan, idx_np, e, w=None):
    exp = R.dispatch_plan(idx_np, e)
    m = idx_np.size
    assert plan.counts.cpu().tolist() == exp["counts"].tolist()
    assert plan.seg.cpu().numpy().tolist() == _seg_expect(exp["counts"], e).tolist()
    assert np.array_equal(plan.dest.cpu().numpy(), exp["dest"])
    assert np.array_equal(plan.row_token.cpu().numpy()[:m], exp["row_token"])
    if w is not None:
        rp = plan.row_prob.cpu().numpy()
        assert np.array_equal(rp, w.reshape(-1)[exp["row_token"] * idx_np.shape[1] + exp["row_slot"]])
    assert int(plan.status.item()) == 0


@pytest.mark.parametrize("t,e,k", [(8192, 128, 8), (256, 8, 2), (1000, 64, 6), (3, 5, 5), (130, 300, 4),
                                   (500, 256, 8), (700, 1024, 32), (0, 128, 8)])
def test_topk_softmax_bit_exact(device, t, e, k):
    ops = _ops()
    print(f"topk t={t} e={e} k={k}", flush=True)
    g = torch.Generator().manual_seed(t + e + k)
    logits = torch.randn(t, e, generator=g)
    if t:
        logits[0, : min(4, e)] = 0.5  # exact ties
    idx, w = ops.router_topk(logits.to(device), k)
    torch.cuda.synchronize()
    exp_idx, exp_w = R.topk_softmax(logits.numpy(), k)
    assert np.array_equal(idx.cpu().numpy(), exp_idx)
    np.testing.assert_allclose(w.cpu().numpy(), exp_w, rtol=2e-6, atol=1e-7)


def test_topk_tie_rule_kats(device):
    ops = _ops()
    for case in KATS["topk_tie_rule"]:
        row = torch.tensor([[float(v) for v in case["logits"]]], dtype=torch.float32)
        idx, _ = ops.router_topk(row.to(device), case["k"])
        assert idx.cpu()[0].tolist() == case["idx"], case
    for case in KATS["softmax_closed_form"]:
        row = torch.tensor([case["logits"]], dtype=torch.float32)
        idx, w = ops.router_topk(row.to(device), case["k"])
        assert idx.cpu()[0].tolist() == case["idx"]
        np.testing.assert_allclose(w.cpu()[0].numpy(), case["w"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", ["replay_bundle_E3_k2", "sampled_bundle_call0", "sampled_bundle_call1"])
def test_replay_and_plan_reference_kats(device, name):
    ops = _ops()
    kat = KATS[name]
    target = torch.tensor(kat["routes"], dtype=torch.int64)
    t, k = target.shape
    e = kat["num_experts"]
    logits = torch.randn(t, e, generator=torch.Generator().manual_seed(3))
    idx, w, status = ops.router_replay(logits.to(device), target.to(device))
    assert int(status.item()) == 0
    assert idx.cpu().tolist() == kat["routes"]
    plan = ops.dispatch_plan(idx, w, e)
    assert plan.counts.cpu().tolist() == kat["counts"]
    assert plan.offsets.cpu().tolist() == kat["offsets"]
    assert plan.row_token.cpu().tolist() == kat["row_token"]
    assert plan.dest.cpu().tolist() == kat["dest"]


def test_replay_zipf_c2_bit_exact(device):
    from art_amd.workloads import CONFIGS, make_inputs
    ops = _ops()
    cfg = CONFIGS["C2"]
    inp = make_inputs(cfg, "cpu", seed=0)
    print("replay C2 full size", flush=True)
    idx, w, status = ops.router_replay(inp.logits.to(device), inp.target.to(device))
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert np.array_equal(idx.cpu().numpy(), inp.target.numpy().astype(np.int32))
    exp_idx, exp_w = R.replay(inp.logits.numpy(), inp.target.numpy())
    np.testing.assert_allclose(w.cpu().numpy(), exp_w, rtol=2e-6, atol=1e-7)
    plan = ops.dispatch_plan(idx, w, cfg.E)
    counts = plan.counts.cpu().numpy()
    assert (counts == 0).any(), "Zipf(1.2) replay should leave some experts empty"
    _check_plan(plan, exp_idx, cfg.E, w.cpu().numpy())


def test_replay_rejects_out_of_range_and_repeated_ids(device):
    ops = _ops()
    logits = torch.randn(3, 4)
    target = torch.tensor([[0, 4], [1, 1], [2, 3]])
    idx, w, status = ops.router_replay(logits.to(device), target.to(device))
    assert int(status.item()) == 2
    assert idx.cpu().tolist() == [[0, -1], [1, -1], [2, 3]]
    assert w.cpu()[0, 1].item() == 0.0 and abs(w.cpu()[0, 0].item() - 1.0) < 1e-6
    plan = ops.dispatch_plan(idx, w, 4)
    assert plan.counts.cpu().tolist() == [1, 1, 1, 1]
    assert plan.dest.cpu().tolist() == [[0, -1], [1, -1], [2, 3]]
    assert int(plan.status.item()) == 2  # the two rejected slots again


@pytest.mark.parametrize("t,e,k", [(8192, 128, 8), (0, 8, 2), (1, 4, 4), (64, 1, 1), (4097, 256, 8),
                                   (3000, 1024, 32)])
def test_dispatch_plan_bit_exact(device, t, e, k):
    ops = _ops()
    print(f"plan t={t} e={e} k={k}", flush=True)
    rng = np.random.default_rng(t * 7 + e)
    idx = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]).astype(np.int32) \
        if t else np.zeros((0, k), np.int32)
    w = rng.random((t, k)).astype(np.float32)
    plan = ops.dispatch_plan(torch.from_numpy(idx).to(device), torch.from_numpy(w).to(device), e)
    torch.cuda.synchronize()
    _check_plan(plan, idx, e, w)


def test_segments_from_counts(device):
    ops = _ops()
    counts = [32, 0, 16, 24, 0, 300, 1]
    seg = ops.segments_from_counts(counts, len(counts), device)
    assert seg.cpu().numpy().tolist() == _seg_expect(counts, len(counts)).tolist()


@pytest.mark.parametrize("t,h,e,k", [(8192, 2048, 128, 8), (33, 256, 8, 2), (5, 8, 4, 3),
                                     (300, 512, 64, 12), (100, 64, 40, 32)])
def test_permute_and_combine_bit_exact(device, t, h, e, k):
    ops = _ops()
    print(f"permute/combine t={t} h={h}", flush=True)
    rng = np.random.default_rng(h)
    idx = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]).astype(np.int32)
    plan = ops.dispatch_plan(torch.from_numpy(idx).to(device), None, e)
    x = torch.randn(t, h, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    xp = ops.permute(x.to(device), plan.dest, t * k)
    exp = R.dispatch_plan(idx, e)
    assert torch.equal(xp.cpu(), x[torch.from_numpy(exp["row_token"])])
    # combine: fp32 sum over j in slot order, rounded once to bf16 -> bit-exact
    yp = torch.randn(t * k, h, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    y = ops.combine(yp.to(device), plan.dest, t)
    dest = torch.from_numpy(exp["dest"])
    acc = torch.zeros(t, h, dtype=torch.float32)
    for j in range(k):
        acc = acc + yp[dest[:, j]].float()
    assert torch.equal(y.cpu(), acc.to(torch.bfloat16))
    # weighted combine: the kernel fuses multiply-add (one rounding), torch rounds
    # the product first, so allow one bf16 ulp
    wgt = torch.rand(t, k, generator=torch.Generator().manual_seed(4))
    y = ops.combine(yp.to(device), plan.dest, t, wgt=wgt.to(device))
    acc = torch.zeros(t, h, dtype=torch.float64)
    for j in range(k):
        acc = acc + wgt[:, j:j + 1].double() * yp[dest[:, j]].double()
    torch.testing.assert_close(y.cpu().double(), acc, rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("k", [8, 12, 20])
def test_combine_router_grad_addend_and_dropped_slots(device, k):
    """Backward combine: sum_j wgt y_perm[dest] + sum_j dl w_r[idx] + addend, with
    some slots dropped (dest = -1), k spanning one to three blocks of 8 slots."""
    ops = _ops()
    print(f"combine backward k={k}", flush=True)
    t, h, e = 200, 256, 48
    g = torch.Generator().manual_seed(k)
    m = t * k
    dest = torch.randperm(m, generator=g).view(t, k).to(torch.int32)
    dest[torch.rand(t, k, generator=g) < 0.1] = -1
    yp = torch.randn(m, h, generator=g).to(torch.bfloat16)
    wgt = torch.rand(t, k, generator=g)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)]).to(torch.int32)
    dl = torch.randn(t, k, generator=g)
    w_r = (torch.randn(e, h, generator=g) * 0.1).to(torch.bfloat16)
    addend = torch.randn(t, h, generator=g).to(torch.bfloat16)
    y = ops.combine(yp.to(device), dest.to(device), t, wgt=wgt.to(device), dl=dl.to(device),
                    idx=idx.to(device), w_r=w_r.to(device), addend=addend.to(device))
    ref = addend.double().clone()
    for j in range(k):
        d = dest[:, j].long()
        ok = (d >= 0).double().unsqueeze(1)
        ref += ok * wgt[:, j:j + 1].double() * yp[d.clamp_min(0)].double()
        ref += dl[:, j:j + 1].double() * w_r[idx[:, j].long()].double()
    torch.testing.assert_close(y.cpu().double(), ref, rtol=2 ** -7, atol=1e-5)


@pytest.mark.parametrize("t,r,e", [(1000, 64, 128), (65, 5, 8), (64, 1, 100), (1, 16, 200),
                                   (300, 256, 64)])
def test_router_lora_apply_matches_fp32(device, t, r, e):
    """logits += s * t_r B (fp32) over ragged token tiles, ranks not a multiple
    of 4 and column counts not a multiple of 64; t_bf16 is t_r rounded once."""
    ops = _ops()
    g = torch.Generator().manual_seed(t + r + e)
    t_r = torch.randn(t, r, generator=g)
    b = (torch.randn(r, e, generator=g) * 0.1).to(torch.bfloat16)
    logits = torch.randn(t, e, generator=g)
    out = logits.to(device)
    t_bf = ops.router_lora_apply(t_r.to(device), b.to(device), out, 0.75, want_bf16=True)
    ref = logits.double() + 0.75 * t_r.double() @ b.double()
    torch.testing.assert_close(out.cpu().double(), ref, rtol=1e-5, atol=1e-5)
    assert torch.equal(t_bf.cpu(), t_r.to(torch.bfloat16))


@pytest.mark.parametrize("t,k,r,e", [(1000, 8, 64, 128), (77, 3, 5, 40), (1, 32, 16, 64),
                                     (130, 20, 100, 300)])
def test_router_lora_grad_matches_fp32(device, t, k, r, e):
    """g = s * dl . B[:, idx] per token and the dense dlogits scatter, with some
    slots dropped (idx = -1), k up to 32 (batches of 64 / k tokens per load)."""
    ops = _ops()
    g0 = torch.Generator().manual_seed(t + k + r)
    idx = torch.stack([torch.randperm(e, generator=g0)[:k] for _ in range(t)]).to(torch.int32)
    idx[torch.rand(t, k, generator=g0) < 0.1] = -1
    dl = torch.randn(t, k, generator=g0)
    b = (torch.randn(r, e, generator=g0) * 0.1).to(torch.bfloat16)
    g, dlog = ops.router_lora_grad(dl.to(device), idx.to(device), b.to(device), 0.5)
    ok = (idx >= 0).double()
    cols = b.double()[:, idx.clamp_min(0).long()]            # [r, t, k]
    g_ref = 0.5 * (cols * (dl.double() * ok).unsqueeze(0)).sum(-1).t()
    dlog_ref = torch.zeros(t, e, dtype=torch.float64)
    for j in range(k):
        sel = idx[:, j] >= 0
        dlog_ref[sel, idx[sel, j].long()] += dl[sel, j].double()
    torch.testing.assert_close(g.cpu().double(), g_ref, rtol=2 ** -7, atol=1e-4)
    torch.testing.assert_close(dlog.cpu().double(), dlog_ref, rtol=2 ** -7, atol=1e-4)


def test_router_replay_rows_equals_gathered_target(device):
    """Replay of table[rows[t]] is bit-exact with replaying the gathered
    target; rows outside the table reject the token's k ids (status counts
    them) like out-of-range ids do."""
    ops = _ops()
    g = torch.Generator().manual_seed(21)
    n, t, e, k = 5000, 3000, 96, 6
    table = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)]).to(torch.int32)
    table[7, 1] = table[7, 0]                       # a repeated id inside one row
    rows = torch.randint(0, n, (t,), generator=g, dtype=torch.int32)
    rows[[3, 10, 2999]] = torch.tensor([-1, n, 7], dtype=torch.int32)
    logits = torch.randn(t, e, generator=g)
    idx_r, w_r, st_r = ops.router_replay_rows(logits.to(device), table.to(device), rows.to(device))
    tgt = table[rows.clamp(0, n - 1).long()].long()
    tgt[3] = -1
    tgt[10] = -1
    idx_t, w_t, st_t = ops.router_replay(logits.to(device), tgt.to(device))
    assert torch.equal(idx_r.cpu(), idx_t.cpu()) and torch.equal(w_r.cpu(), w_t.cpu())
    assert int(st_r.item()) == int(st_t.item()) == 2 * k + 1
    assert (idx_r[3] == -1).all() and (idx_r[10] == -1).all() and int(idx_r[2999, 1]) == -1


def test_router_replay_rows_reads_the_side_table_for_negative_rows(device):
    """rows[t] < 0 replays extra[-rows[t] - 1] (the synthetic rows of tokens
    without a captured route); entries past the side table are rejected."""
    ops = _ops()
    g = torch.Generator().manual_seed(22)
    n, x, t, e, k = 300, 5, 200, 64, 8
    table = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)]).to(torch.int32)
    extra = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(x)]).to(torch.int32)
    rows = torch.randint(0, n, (t,), generator=g, dtype=torch.int32)
    rows[[0, 17, 60, 199]] = torch.tensor([-1, -5, -3, -6], dtype=torch.int32)   # -6: past extra
    logits = torch.randn(t, e, generator=g)
    idx, w, st = ops.router_replay_rows(logits.to(device), table.to(device), rows.to(device),
                                        extra=extra.to(device))
    tgt = torch.where(rows.unsqueeze(1) >= 0, table[rows.clamp(0, n - 1).long()],
                      extra[(-rows - 1).clamp(0, x - 1).long()]).long()
    tgt[199] = -1
    idx_t, w_t, st_t = ops.router_replay(logits.to(device), tgt.to(device))
    assert torch.equal(idx.cpu(), idx_t.cpu()) and torch.equal(w.cpu(), w_t.cpu())
    assert int(st.item()) == int(st_t.item()) == k
    assert idx[17].tolist() == extra[4].tolist() and idx[0].tolist() == extra[0].tolist()
