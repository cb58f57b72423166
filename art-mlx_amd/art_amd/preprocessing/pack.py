"""Packing tokenised results into fixed-length rows with prefix-tree sharing,
carrying each token's captured MoE route into the packed layout.

Mirrors the route-relevant part of ``art.preprocessing.pack``
(/root/reference/src/art/preprocessing/pack.py:78-423) and the radix packing
of ``art.megatron.prefix_tree_packing`` (/root/reference/src/art/megatron/
prefix_tree_packing.py:27-256): the packed layout (shared prompt segments
written once, then each branch; ``group_ids`` per emitted segment counting
from 1, ``parent_ids`` pointing at the segment continued, roots at
themselves), which tokens may be shared (``shareable_length`` = the prompt up
to the token before the first trainable one), the padding values, the
advantage / weight normalisation and the route statistics are format and stay
as they are.  Images are not carried (not part of the MoE path).

How it works here.  The prefix tree is planned over Python int tuples with an
explicit work stack (no recursion limit on deep trees).  The shared prefix of
a group is found by comparing its lexicographically smallest and largest
member (every member agrees wherever those two do).  Routes are written into
the packed row in one pass per sequence; positions a later sequence shares
count slot conflicts against the route already there.
"""
from __future__ import annotations

import math
import random
from dataclasses import dataclass, field
from typing import Any

import torch

from .moe_routing import (MoeRoutingPackStats, PackedMoeRoutingReplay, TokenRoute,
                          count_route_slot_conflicts, tensorize_moe_routes)


@dataclass
class TokenizedResult:
    """The fields of a tokenised trajectory the packer reads (the reference's
    ``TokenizedResult`` carries more; the packer touches only these)."""
    token_ids: list[int]
    input_pos: list[int]
    assistant_mask: list[int]
    logprobs: list[float]
    advantage: float = 0.0
    weight: float = 1.0
    prompt_id: int = 0
    prompt_length: int = 0
    moe_routed_experts: list[TokenRoute | None] | None = None
    choice_offsets: list[int] = field(default_factory=list)


# ----------------------------------------------------------- prefix tree plan
@dataclass(frozen=True)
class Segment:
    sequences: tuple[int, ...]   # sequences whose tokens [start, end) this segment holds
    start: int
    end: int
    group_id: int
    parent_id: int


def plan_prefix_tree(rows: list[tuple[int, ...]], *, max_depth: int,
                     shareable: list[int]) -> list[Segment]:
    """Segments of the packed layout, in emission order.  A group of
    sequences that may still share (``shareable[i] > start``) writes its
    common prefix once and continues below it; members that may not share,
    single members, and branches deeper than ``max_depth`` (0: no sharing)
    are written as tails.  Members without a common next token split by that
    token, in first-seen order."""
    if max_depth < 0:
        raise ValueError("max_depth must be >= 0")
    lens = [len(r) for r in rows]
    segments: list[Segment] = []

    def emit(seqs: tuple[int, ...], start: int, end: int, parent: int | None) -> int:
        gid = len(segments) + 1
        segments.append(Segment(seqs, start, end, gid, gid if parent is None else parent))
        return gid

    # work items: (members, start, parent group, depth); a stack popped LIFO,
    # so children are pushed in reverse to keep first-seen order
    stack: list[tuple[tuple[int, ...], int, int | None, int]] = [
        (tuple(range(len(rows))), 0, None, 0)]
    while stack:
        members, start, parent, depth = stack.pop()
        live = [i for i in members if lens[i] > start]
        share = tuple(i for i in live if shareable[i] > start)
        for i in live:
            if shareable[i] <= start:
                emit((i,), start, lens[i], parent)
        if not share:
            continue
        if max_depth == 0 or len(share) == 1 or (parent is not None and depth >= max_depth):
            for i in share:
                emit((i,), start, lens[i], parent)
            continue
        limit = min(min(lens[i], shareable[i]) for i in share)
        lo = min(rows[i] for i in share)
        hi = max(rows[i] for i in share)
        end = start
        while end < limit and lo[end] == hi[end]:
            end += 1
        if end > start:
            gid = emit(share, start, end, parent)
            stack.append((share, end, gid, depth + 1))
            continue
        branches: dict[int, list[int]] = {}
        for i in share:
            branches.setdefault(rows[i][start], []).append(i)
        for group in reversed(list(branches.values())):
            stack.append((tuple(group), start, parent, depth))
    return segments


def packed_token_count(rows: list[tuple[int, ...]], *, max_depth: int,
                       shareable: list[int]) -> int:
    return sum(s.end - s.start for s in plan_prefix_tree(rows, max_depth=max_depth,
                                                         shareable=shareable))


# ------------------------------------------------------------------- packing
def _first_trainable(r: TokenizedResult) -> int:
    for i, (m, lp) in enumerate(zip(r.assistant_mask, r.logprobs, strict=True)):
        if m or not math.isnan(float(lp)):
            return i
    return len(r.token_ids)


@dataclass
class _Item:
    tokens: tuple[int, ...]
    input_pos: tuple[int, ...]
    mask: tuple[int, ...]
    logprobs: tuple[float, ...]
    advantage: float
    weight: float
    shareable: int
    routes: tuple[TokenRoute | None, ...] | None

    def truncated(self, n: int) -> "_Item":
        if len(self.tokens) <= n:
            return self
        return _Item(self.tokens[:n], self.input_pos[:n], self.mask[:n], self.logprobs[:n],
                     self.advantage, self.weight, min(self.shareable, n),
                     None if self.routes is None else self.routes[:n])


def _item(r: TokenizedResult, seq_len: int) -> _Item:
    share = min(int(r.prompt_length), max(_first_trainable(r) - 1, 0))
    return _Item(tuple(int(t) for t in r.token_ids), tuple(int(p) for p in r.input_pos),
                 tuple(int(m) for m in r.assistant_mask), tuple(float(v) for v in r.logprobs),
                 float(r.advantage), float(r.weight), share,
                 None if r.moe_routed_experts is None else tuple(r.moe_routed_experts)
                 ).truncated(seq_len)


def _pack_row(row: list[_Item], seq_len: int, pack: bool, with_routes: bool,
              stats: MoeRoutingPackStats) -> dict[str, list]:
    segs = plan_prefix_tree([it.tokens for it in row], max_depth=seq_len if pack else 0,
                            shareable=[it.shareable if pack else 0 for it in row])
    n = sum(s.end - s.start for s in segs)
    tokens, gids, pids = [0] * n, [0] * n, [0] * n
    where: list[list[int]] = [[] for _ in row]       # packed position of each source token
    cur = 0
    for s in segs:
        src = row[s.sequences[0]].tokens
        for j in range(s.end - s.start):
            tokens[cur + j] = src[s.start + j]
            gids[cur + j], pids[cur + j] = s.group_id, s.parent_id
        for i in s.sequences:
            where[i].extend(range(cur, cur + s.end - s.start))
        cur += s.end - s.start
    taken = [False] * n
    pos, mask, lps = [0] * n, [0] * n, [float("nan")] * n
    adv, wts = [0.0] * n, [0.0] * n
    routes: list[TokenRoute | None] = [None] * n
    for it, places in zip(row, where):
        for si, p in enumerate(places):
            if tokens[p] != it.tokens[si]:
                raise RuntimeError("Prefix-tree pack token assignment mismatch")
            route = it.routes[si] if it.routes is not None and si < len(it.routes) else None
            if taken[p]:
                if pos[p] != it.input_pos[si]:
                    raise RuntimeError("Prefix-tree pack cannot share mismatched input positions")
                if it.mask[si] or not math.isnan(it.logprobs[si]):
                    raise RuntimeError("Prefix-tree pack attempted to share a trainable token")
                if with_routes:
                    if routes[p] is None or route is None:
                        raise RuntimeError("Prefix-tree MoE route is missing")
                    compared, conflicts = count_route_slot_conflicts(routes[p], route)
                    stats.prefix_tree_rows += 1
                    stats.prefix_tree_compared_slots += compared
                    stats.prefix_tree_conflict_slots += conflicts
                    stats.prefix_tree_conflict_rows += int(conflicts > 0)
                continue
            taken[p] = True
            pos[p], mask[p], lps[p] = it.input_pos[si], it.mask[si], it.logprobs[si]
            adv[p], wts[p] = it.advantage, it.weight
            routes[p] = route
    cut = slice(0, seq_len)
    return {"token_ids": tokens[cut], "group_ids": gids[cut], "parent_ids": pids[cut],
            "input_pos": pos[cut], "assistant_mask": mask[cut], "logprobs": lps[cut],
            "advantages": adv[cut], "weights": wts[cut],
            "moe_routes": routes[cut] if with_routes else []}


def packed_tensors_from_tokenized_results(
        tokenized_results: list[TokenizedResult], seq_len: int, pad_token_id: int = -100,
        truncate_long_results: bool = True, advantage_balance: float = 0.0, verbosity: int = 1,
        pack_results: bool = True, include_moe_routing: bool = False) -> dict[str, Any]:
    """Rows of at most ``seq_len`` packed tokens (results are appended to the
    current row while its packed size fits; rows are shuffled), with
    ``moe_routing_replay`` (a PackedMoeRoutingReplay) when
    ``include_moe_routing`` asks for the captured routes."""
    rows: list[list[_Item]] = [[]]
    stats = MoeRoutingPackStats()
    for r in tokenized_results:
        if len(r.token_ids) > seq_len and not truncate_long_results:
            if verbosity > 1:
                print("Result is too long, skipping")
            continue
        if include_moe_routing and r.moe_routed_experts is None:
            raise RuntimeError("MoE routing replay from trajectories was requested, but a "
                               "tokenized result has no aligned routed experts")
        if sum(r.assistant_mask[r.prompt_length:]) == 0:
            if verbosity > 1:
                print("Result has no unique completion tokens, skipping")
            continue
        it = _item(r, seq_len)
        if rows[-1]:
            cand = rows[-1] + [it]
            size = packed_token_count([c.tokens for c in cand], max_depth=seq_len,
                                      shareable=[c.shareable for c in cand])
            if not pack_results or size > seq_len:
                rows.append([])
        rows[-1].append(it)
    random.shuffle(rows)
    packed = [_pack_row(row, seq_len, pack_results, include_moe_routing, stats) if row else
              {k: [] for k in ("token_ids", "group_ids", "parent_ids", "input_pos",
                               "assistant_mask", "logprobs", "advantages", "weights",
                               "moe_routes")}
              for row in rows]

    def col(name: str, pad: Any) -> list[list]:
        return [r[name] + [pad] * (seq_len - len(r[name])) for r in packed]

    mask = torch.tensor(col("assistant_mask", 0), dtype=torch.bool)
    weights = torch.where(mask, torch.tensor(col("weights", 0.0)), 0.0)
    weights[mask] /= weights[mask].mean()
    adv = torch.where(mask, torch.tensor(col("advantages", 0.0)), 0.0)
    if advantage_balance > 0.0:
        adv = torch.where(adv > 0, adv, adv * (1 - advantage_balance))
    elif advantage_balance < 0.0:
        adv = torch.where(adv < 0, adv, adv * (1 + advantage_balance))
    adv[mask] /= (adv[mask].abs() * weights[mask]).mean()
    out: dict[str, Any] = {
        "tokens": torch.tensor(col("token_ids", pad_token_id)),
        "group_ids": torch.tensor(col("group_ids", -1)),
        "parent_ids": torch.tensor(col("parent_ids", -1)),
        "input_pos": torch.tensor(col("input_pos", 0)),
        "assistant_mask": mask,
        "logprobs": torch.tensor(col("logprobs", float("nan"))),
        "advantages": adv,
        "weights": weights,
        "moe_routing_replay": None,
    }
    if include_moe_routing:
        idx, tmask, n_layers, k, n_exp = tensorize_moe_routes([r["moe_routes"] for r in packed],
                                                               seq_len)
        stats.packed_tokens = int(tmask.sum())
        out["moe_routing_replay"] = PackedMoeRoutingReplay(
            expert_indices=idx, token_mask=tmask, num_layers=n_layers, topk=k, num_experts=n_exp,
            pack_stats=stats)
    return out
