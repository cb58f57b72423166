"""MoE routing replay: bundle format, bundle builder and the per-call controller.

Host-side counterpart of /root/reference/src/art/megatron/routing_replay.py.
A *bundle* holds, for every training step, router and router call, the top-k
expert ids the inference engine chose for each token; the *controller* maps
the tokens of the local micro-batch (by global token uid) to bundle rows and
hands the router a ``[T_local, k]`` int64 target that replaces top-k
selection.  On this build the target feeds ``ops.router_replay`` (the HIP
gather + softmax kernel) through :class:`RouterReplay` / :class:`TopKRouter`,
or ``moe_lora_layer(..., target=...)`` directly.

On-disk format (identical to the reference, routing_replay.py:369-462):
  manifest.json            format_version "moe_routing_replay_v2", topology,
                           num_steps, max_topk, router_keys, steps{step: {file,
                           routers{router_key: {call: {num_experts, sample_index?,
                           micro_slot?, rank_token_counts?}}}}}
  step_%06d.safetensors    "global_token_uids" int64 [N] and, per call,
                           "{router_key}/call_{i}/expert_indices" int32 [N,k],
                           ".../expert_probs" fp32 [N,k] (optional),
                           ".../expert_mask" bool [N,k]

Synthetic rows (tokens with no captured route) use Python's stdlib
``random.Random(seed + (pos + 1) * 1_299_709).sample(range(E), k)`` with the
reference's seed formulas (routing_replay.py:538-539, 553-555, 594-610,
1467-1472), so bundles and targets built here match the reference's bit for
bit.

Parallel topology enters only through a ``parallel_state``-like object
(tensor/context/data-parallel world sizes and ranks); the default is a single
process (all sizes 1), which is what one GPU runs.
"""
from __future__ import annotations

import enum
import json
import logging
import math
import os
import random
import re
import types
import weakref
from collections import defaultdict
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Callable, Iterable, Mapping

import torch

ROUTER_NAME_TOKEN = ".mlp.router"
ROUTER_KEY_FORMAT_VERSION = "moe_routing_replay_v2"
GLOBAL_TOKEN_UIDS_KEY = "global_token_uids"

# seed constants of the synthetic-row generator (routing_replay.py:538-539, 553-555, 605, 1471)
_SEED_SAMPLE = 1_000_003
_SEED_LAYER = 97_003
_SEED_SLOT = 9_176
_SEED_POSITION = 1_299_709

_LAYER_RE = re.compile(r"decoder\.layers\.(?P<layer>\d+)\.mlp\.router$")
_CHUNK_RE = re.compile(r"^chunk(?P<chunk>\d+)\.(?P<name>.+)$")
logger = logging.getLogger(__name__)

_active_controller: "MoeRoutingReplayController | None" = None


def active_routing_replay_controller() -> "MoeRoutingReplayController | None":
    """The controller whose router patches are installed, if any."""
    return _active_controller


# --------------------------------------------------------------------- names
_FUSED_PAIRS = {"linear_proj", "linear_qkv", "in_proj", "linear_fc1", "linear_fc2"}


def canonical_module_name(name: str) -> str:
    """Drop wrapper segments from a module path: leading ``module.``, every
    ``_orig_mod`` (torch.compile), doubled fused-linear names and the
    row-parallel LoRA wrapper (param_name_canonicalization.py:17-54)."""
    parts = name.split(".")
    while parts and parts[0] == "module":
        parts.pop(0)
    out: list[str] = []
    i = 0
    while i < len(parts):
        cur = parts[i]
        nxt = parts[i + 1] if i + 1 < len(parts) else None
        if cur == "_orig_mod":
            i += 1
        elif nxt is not None and cur in _FUSED_PAIRS and nxt == cur:
            out.append(cur)
            i += 2
        elif nxt == "linear_proj" and cur == "out_proj":
            out.append(cur)
            i += 2
        elif nxt == "linear_proj" and cur == "row_parallel_lora":
            i += 2
        else:
            out.append(cur)
            i += 1
    return ".".join(out)


def build_router_key_from_module_name(*, chunk_index: int, module_name: str) -> str:
    """``chunk_{cc}.layer_{llll}.mlp.router`` (routing_replay.py:89-100)."""
    canonical = canonical_module_name(module_name)
    m = _LAYER_RE.search(canonical)
    if m is None:
        raise RuntimeError(
            f"Unable to derive router key from module name '{module_name}'. "
            f"Canonicalized to '{canonical}', expected suffix matching '{_LAYER_RE.pattern}'.")
    return f"chunk_{chunk_index:02d}.layer_{int(m.group('layer')):04d}.mlp.router"


def build_router_key_from_trace_name(trace_module_name: str) -> str:
    """Router key from a ``chunk<idx>.<module name>`` trace name (routing_replay.py:103-115)."""
    m = _CHUNK_RE.match(trace_module_name)
    if m is None:
        raise RuntimeError("Forward trace router module name must start with 'chunk<idx>.'; "
                           f"got '{trace_module_name}'")
    return build_router_key_from_module_name(chunk_index=int(m.group("chunk")),
                                             module_name=m.group("name"))


# -------------------------------------------------------------- bundle types
def _cpu(t: Any, dtype: torch.dtype) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"Expected torch.Tensor, got {type(t)}")
    return t.detach().to(device="cpu", dtype=dtype).contiguous()


@dataclass
class ParallelTopology:
    """Parallel layout the routes were captured under (routing_replay.py:118-126)."""
    tp: int
    ep: int
    etp: int = 1
    dp: int = 1
    sp: bool = False
    cp: int = 1
    pp: int = 1
    vpp: int = 1

    def to_json(self) -> dict[str, Any]:
        return {"tp": self.tp, "ep": self.ep, "etp": self.etp, "dp": self.dp, "sp": self.sp,
                "cp": self.cp, "pp": self.pp, "vpp": self.vpp}

    @classmethod
    def from_json(cls, d: Mapping[str, Any]) -> "ParallelTopology":
        fields = ("tp", "ep", "etp", "dp", "sp", "cp", "pp", "vpp")
        return cls(**{k: d[k] for k in fields if k in d})


def parallel_topology_from_env() -> ParallelTopology:
    """Topology from the ART_MEGATRON_* environment (routing_replay.py:577-587)."""
    def env(name: str, default: int) -> int:
        raw = os.environ.get(name)
        return default if raw in (None, "") else int(raw)
    tp = env("ART_MEGATRON_TENSOR_MODEL_PARALLEL_SIZE", 1)
    etp = env("ART_MEGATRON_EXPERT_TENSOR_PARALLEL_SIZE",
              env("ART_MEGATRON_EXPERT_TENSOR_MODEL_PARALLEL_SIZE", 1))
    return ParallelTopology(tp=tp, ep=env("ART_MEGATRON_EXPERT_MODEL_PARALLEL_SIZE", 1), etp=etp,
                            dp=1, sp=tp > 1, cp=env("ART_MEGATRON_CONTEXT_PARALLEL_SIZE", 1),
                            pp=env("ART_MEGATRON_PIPELINE_MODEL_PARALLEL_SIZE", 1))


@dataclass
class RouterCallRoute:
    """Routes of one router call: int32 ids [N,k], optional fp32 probs, bool
    mask (must be all true), and the micro-batch it belongs to
    (routing_replay.py:125-218)."""
    expert_indices: torch.Tensor
    expert_mask: torch.Tensor
    num_experts: int
    expert_probs: torch.Tensor | None = None
    sample_index: int | None = None
    micro_slot: int | None = None
    rank_token_counts: tuple[int, ...] | None = None

    def __post_init__(self) -> None:
        self.expert_indices = _cpu(self.expert_indices, torch.int32)
        if self.expert_probs is not None:
            self.expert_probs = _cpu(self.expert_probs, torch.float32)
        self.expert_mask = _cpu(self.expert_mask, torch.bool)
        idx = self.expert_indices
        if idx.ndim != 2:
            raise RuntimeError(
                f"expert_indices must have shape [num_tokens, topk], got {tuple(idx.shape)}")
        if self.expert_probs is not None and self.expert_probs.shape != idx.shape:
            raise RuntimeError("expert_probs shape must match expert_indices shape, got "
                               f"{tuple(self.expert_probs.shape)} vs {tuple(idx.shape)}")
        if self.expert_mask.shape != idx.shape:
            raise RuntimeError("expert_mask shape must match expert_indices shape, got "
                               f"{tuple(self.expert_mask.shape)} vs {tuple(idx.shape)}")
        if not bool(self.expert_mask.all()):
            raise RuntimeError(
                "masked slots are unsupported by Megatron native MoE routing replay; route "
                "bundles must contain a valid full top-k expert id row for every replayed token")
        self.num_experts = int(self.num_experts)
        if self.num_experts <= 0:
            raise RuntimeError(f"num_experts must be >0, got {self.num_experts}")
        if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= self.num_experts):
            raise RuntimeError("expert_indices contain ids outside [0, num_experts): "
                               f"num_experts={self.num_experts}")
        if self.sample_index is not None:
            self.sample_index = int(self.sample_index)
        if self.micro_slot is not None:
            self.micro_slot = int(self.micro_slot)
        if self.rank_token_counts is not None:
            counts = tuple(int(c) for c in self.rank_token_counts)
            if any(c < 0 for c in counts):
                raise RuntimeError(f"rank_token_counts must be non-negative, got {counts}")
            if sum(counts) != idx.shape[0]:
                raise RuntimeError("rank_token_counts must sum to route token count: "
                                   f"counts={counts}, tokens={idx.shape[0]}")
            self.rank_token_counts = counts

    @property
    def num_global_tokens(self) -> int:
        return int(self.expert_indices.shape[0])

    @property
    def max_topk(self) -> int:
        return int(self.expert_indices.shape[1])

    @property
    def call_key(self) -> tuple[str, int] | None:
        """Which micro-batch the call belongs to: a sample, a dummy micro slot, or unknown."""
        if self.sample_index is not None:
            return ("sample", self.sample_index)
        if self.micro_slot is not None:
            return ("dummy_micro_slot", self.micro_slot)
        return None


@dataclass
class StepRouterRoutes:
    calls: dict[int, RouterCallRoute]

    def __post_init__(self) -> None:
        if not self.calls:
            raise RuntimeError("StepRouterRoutes.calls cannot be empty")
        for ci in self.calls:
            if ci < 0:
                raise RuntimeError(f"call_index must be >=0, got {ci}")


@dataclass
class StepRoutes:
    """All routers of one step plus the step's global token uids (routing_replay.py:221-285)."""
    routers: dict[str, StepRouterRoutes]
    global_token_uids: torch.Tensor

    def __post_init__(self) -> None:
        if not self.routers:
            raise RuntimeError("StepRoutes.routers cannot be empty")
        uids = _cpu(self.global_token_uids, torch.int64)
        self.global_token_uids = uids
        if uids.ndim != 1:
            raise RuntimeError("global_token_uids must have shape [num_global_tokens], got "
                               f"{tuple(uids.shape)}")
        if torch.unique(uids).numel() != uids.numel():
            raise RuntimeError("global_token_uids must be unique per step")
        n = uids.numel()
        per_micro: dict[tuple[str, int], int] = {}
        for rk, rr in self.routers.items():
            for ci, route in rr.calls.items():
                key = route.call_key
                tokens = route.num_global_tokens
                if key is None:
                    if tokens != n:
                        raise RuntimeError(
                            "Route token count must match step global_token_uids when no "
                            f"per-micro metadata is present: router='{rk}', call={ci}, "
                            f"route_tokens={tokens}, global_token_uids={n}")
                    continue
                if tokens > n:
                    raise RuntimeError(
                        "Route token count exceeds step global_token_uids span: "
                        f"router='{rk}', call={ci}, call_key={key}, route_tokens={tokens}, "
                        f"global_token_uids={n}")
                seen = per_micro.setdefault(key, tokens)
                if seen != tokens:
                    raise RuntimeError(
                        "Route token count must be consistent for the same micro: "
                        f"router='{rk}', call={ci}, call_key={key}, expected={seen}, got={tokens}")


def _key(router_key: str, call_index: int, name: str) -> str:
    return f"{router_key}/call_{call_index}/{name}"


@dataclass
class MoeRoutingReplayBundle:
    """Routes for ``num_steps`` steps (routing_replay.py:288-462)."""
    topology: ParallelTopology
    num_steps: int
    max_topk: int
    router_keys: list[str]
    steps: dict[int, StepRoutes]
    format_version: str = ROUTER_KEY_FORMAT_VERSION

    def __post_init__(self) -> None:
        if self.format_version != ROUTER_KEY_FORMAT_VERSION:
            raise RuntimeError(f"Unsupported MoE routing replay bundle format: "
                               f"{self.format_version!r}; expected {ROUTER_KEY_FORMAT_VERSION!r}")
        if self.num_steps <= 0:
            raise RuntimeError(f"num_steps must be >0, got {self.num_steps}")
        if self.max_topk <= 0:
            raise RuntimeError(f"max_topk must be >0, got {self.max_topk}")
        if not self.router_keys:
            raise RuntimeError("router_keys cannot be empty")
        if len(set(self.router_keys)) != len(self.router_keys):
            raise RuntimeError("router_keys must be unique")
        want = set(range(self.num_steps))
        if set(self.steps) != want:
            raise RuntimeError(f"steps must contain exactly {sorted(want)}, got {sorted(self.steps)}")
        keys = set(self.router_keys)
        for si, sr in self.steps.items():
            if set(sr.routers) != keys:
                raise RuntimeError(f"Step {si} router keys differ from bundle router keys: "
                                   f"step_keys={sorted(sr.routers)}, router_keys={self.router_keys}")
            for rr in sr.routers.values():
                for route in rr.calls.values():
                    if route.max_topk > self.max_topk:
                        raise RuntimeError("Route topk exceeds bundle max_topk: "
                                           f"route_topk={route.max_topk}, max_topk={self.max_topk}")

    # ------------------------------------------------------------ disk I/O
    @classmethod
    def from_dir(cls, bundle_dir: str | Path) -> "MoeRoutingReplayBundle":
        from safetensors.torch import load_file

        base = Path(bundle_dir)
        mpath = base / "manifest.json"
        if not mpath.exists():
            raise FileNotFoundError(f"Missing routing replay manifest: {mpath}")
        manifest = json.loads(mpath.read_text(encoding="utf-8"))
        if manifest.get("format_version") != ROUTER_KEY_FORMAT_VERSION:
            raise RuntimeError(f"Unsupported MoE routing replay bundle format: "
                               f"{manifest.get('format_version')!r}; expected "
                               f"{ROUTER_KEY_FORMAT_VERSION!r}")
        steps: dict[int, StepRoutes] = {}
        for step_str, info in manifest["steps"].items():
            si = int(step_str)
            # clone: own the storage instead of keeping the file mapped
            tensors = {k: v.clone().contiguous() for k, v in load_file(str(base / info["file"])).items()}
            if GLOBAL_TOKEN_UIDS_KEY not in tensors:
                raise RuntimeError(f"Missing tensor key '{GLOBAL_TOKEN_UIDS_KEY}' for step={si}")
            routers: dict[str, StepRouterRoutes] = {}
            for rk, calls_info in info["routers"].items():
                calls: dict[int, RouterCallRoute] = {}
                for ci_str, ci_info in calls_info.items():
                    ci = int(ci_str)
                    need = [_key(rk, ci, "expert_indices"), _key(rk, ci, "expert_mask")]
                    missing = [k for k in need if k not in tensors]
                    if missing:
                        raise RuntimeError(f"Missing tensor keys {missing} in {info['file']}")
                    calls[ci] = RouterCallRoute(
                        expert_indices=tensors[need[0]], expert_mask=tensors[need[1]],
                        expert_probs=tensors.get(_key(rk, ci, "expert_probs")),
                        num_experts=int(ci_info["num_experts"]),
                        sample_index=ci_info.get("sample_index"),
                        micro_slot=ci_info.get("micro_slot"),
                        rank_token_counts=ci_info.get("rank_token_counts"))
                routers[rk] = StepRouterRoutes(calls=calls)
            steps[si] = StepRoutes(routers=routers, global_token_uids=tensors[GLOBAL_TOKEN_UIDS_KEY])
        return cls(format_version=manifest["format_version"],
                   topology=ParallelTopology.from_json(manifest["topology"]),
                   num_steps=int(manifest["num_steps"]), max_topk=int(manifest["max_topk"]),
                   router_keys=list(manifest["router_keys"]), steps=steps)

    def to_dir(self, bundle_dir: str | Path) -> None:
        from safetensors.torch import save_file

        base = Path(bundle_dir)
        base.mkdir(parents=True, exist_ok=True)
        steps_manifest: dict[str, Any] = {}
        for si in sorted(self.steps):
            sr = self.steps[si]
            if si < 0:
                raise ValueError(f"step_index must be non-negative, got {si}")
            fname = f"step_{si:06d}.safetensors"
            tensors: dict[str, torch.Tensor] = {GLOBAL_TOKEN_UIDS_KEY: sr.global_token_uids}
            routers_manifest: dict[str, Any] = {}
            for rk in sorted(sr.routers):
                calls_manifest: dict[str, Any] = {}
                for ci in sorted(sr.routers[rk].calls):
                    route = sr.routers[rk].calls[ci]
                    tensors[_key(rk, ci, "expert_indices")] = route.expert_indices
                    if route.expert_probs is not None:
                        tensors[_key(rk, ci, "expert_probs")] = route.expert_probs
                    tensors[_key(rk, ci, "expert_mask")] = route.expert_mask
                    meta: dict[str, Any] = {"num_experts": route.num_experts}
                    if route.sample_index is not None:
                        meta["sample_index"] = route.sample_index
                    if route.micro_slot is not None:
                        meta["micro_slot"] = route.micro_slot
                    if route.rank_token_counts is not None:
                        meta["rank_token_counts"] = list(route.rank_token_counts)
                    calls_manifest[str(ci)] = meta
                routers_manifest[rk] = calls_manifest
            save_file(tensors, str(base / fname))
            steps_manifest[str(si)] = {"file": fname, "routers": routers_manifest}
        manifest = {"format_version": self.format_version, "topology": self.topology.to_json(),
                    "num_steps": self.num_steps, "max_topk": self.max_topk,
                    "router_keys": self.router_keys, "steps": steps_manifest}
        (base / "manifest.json").write_text(json.dumps(manifest, indent=2, sort_keys=True),
                                            encoding="utf-8")


# ------------------------------------------------------------ synthetic rows
def synthetic_replay_rows(*, row_positions: torch.Tensor | Iterable[int], num_experts: int,
                          topk: int, dtype: torch.dtype, seed: int) -> torch.Tensor:
    """k distinct expert ids per position, ``random.Random(seed + (pos+1)*1_299_709)
    .sample(range(E), k)`` (routing_replay.py:594-610)."""
    pos = row_positions.tolist() if isinstance(row_positions, torch.Tensor) else list(row_positions)
    rows = [random.Random(seed + (int(p) + 1) * _SEED_POSITION).sample(range(num_experts), topk)
            for p in pos]
    if not rows:
        return torch.empty((0, topk), dtype=dtype)
    return torch.tensor(rows, dtype=dtype)


_synthetic_replay_rows = synthetic_replay_rows


# ------------------------------------------------------------------ builder
def _rows_without_future_scored_tokens(group_ids: torch.Tensor, parent_ids: torch.Tensor,
                                       logprobs: torch.Tensor) -> torch.Tensor:
    """Branch rows after which no token of the same group is scored: their
    route cannot influence a trained token (routing_replay.py:38-68)."""
    valid = group_ids != -1
    branch = valid & (group_ids != parent_ids)
    scored = valid & torch.isfinite(logprobs)
    out = torch.zeros_like(branch)
    g = group_ids.tolist()
    br = branch.tolist()
    sc = scored.tolist()
    for s in range(len(g)):
        scored_later: set[int] = set()
        for p in range(len(g[s]) - 1, -1, -1):
            gid = g[s][p]
            if gid == -1:
                continue
            out[s, p] = br[s][p] and gid not in scored_later
            if sc[s][p]:
                scored_later.add(gid)
    return out


def build_moe_routing_replay_bundle_from_packed_tensors(
        *, packed_tensors: Mapping[str, Any], global_grad_accumulation_sequences: int,
        topology: ParallelTopology | None = None) -> MoeRoutingReplayBundle:
    """One step per ``global_grad_accumulation_sequences`` packed sequences, one
    router key per layer, one call per sequence (routing_replay.py:465-574).

    ``packed_tensors["moe_routing_replay"]`` carries ``expert_indices``
    [S, seq, L, k], ``token_mask`` [S, seq] (route captured) and ``num_experts``;
    ``group_ids``, ``parent_ids`` and ``logprobs`` [S, seq] decide which missing
    routes are tolerated (padding, terminal completion tokens, branch tails
    with no later scored token) and get synthetic rows.  Step slots past the
    last sequence become dummy micro slots with synthetic routes.
    """
    rr = packed_tensors.get("moe_routing_replay")
    if rr is None:
        raise RuntimeError("Packed tensors do not contain MoE routing replay data")
    if global_grad_accumulation_sequences <= 0:
        raise RuntimeError("global_grad_accumulation_sequences must be positive when building MoE "
                           f"routing replay bundles, got {global_grad_accumulation_sequences}")
    idx = rr.expert_indices
    token_mask = rr.token_mask
    n_seq, seq_len, n_layers, topk = (int(d) for d in idx.shape)
    n_exp = int(rr.num_experts)
    gid = packed_tensors["group_ids"]
    pid = packed_tensors["parent_ids"]
    valid = gid != -1
    next_gid = torch.cat([gid[:, 1:], torch.full_like(gid[:, :1], -1)], dim=1)
    terminal = valid & (gid != pid) & (gid != next_gid)
    tolerated = terminal | _rows_without_future_scored_tokens(gid, pid, packed_tensors["logprobs"])
    bad = valid & ~token_mask & ~tolerated
    if bool(bad.any()):
        raise RuntimeError("Packed tensors are missing MoE routes outside terminal completion "
                           f"tokens: missing_rows={int(bad.sum())}")
    keys = [f"chunk_00.layer_{layer:04d}.mlp.router" for layer in range(n_layers)]
    gga = global_grad_accumulation_sequences
    n_steps = math.ceil(n_seq / gga)
    steps: dict[int, StepRoutes] = {}
    ones = lambda t: torch.ones_like(t, dtype=torch.bool)  # noqa: E731
    for step in range(n_steps):
        routers: dict[str, StepRouterRoutes] = {}
        for layer, rk in enumerate(keys):
            calls: dict[int, RouterCallRoute] = {}
            for slot in range(gga):
                sample = step * gga + slot
                if sample < n_seq:
                    rows = idx[sample, :, layer, :].clone()
                    missing = ~token_mask[sample]
                    if bool(missing.any()):
                        rows[missing] = synthetic_replay_rows(
                            row_positions=torch.nonzero(missing).flatten(), num_experts=n_exp,
                            topk=topk, dtype=idx.dtype,
                            seed=(sample + 1) * _SEED_SAMPLE + (layer + 1) * _SEED_LAYER)
                    calls[slot] = RouterCallRoute(expert_indices=rows, expert_mask=ones(rows),
                                                  num_experts=n_exp, sample_index=sample)
                else:
                    rows = synthetic_replay_rows(
                        row_positions=range(seq_len), num_experts=n_exp, topk=topk,
                        dtype=idx.dtype,
                        seed=(step + 1) * _SEED_SAMPLE + (layer + 1) * _SEED_LAYER
                        + (slot + 1) * _SEED_SLOT)
                    calls[slot] = RouterCallRoute(expert_indices=rows, expert_mask=ones(rows),
                                                  num_experts=n_exp, micro_slot=slot)
            routers[rk] = StepRouterRoutes(calls=calls)
        steps[step] = StepRoutes(routers=routers,
                                 global_token_uids=torch.arange(seq_len, dtype=torch.int64))
    return MoeRoutingReplayBundle(topology=topology or parallel_topology_from_env(),
                                  num_steps=n_steps, max_topk=topk, router_keys=keys, steps=steps)


# ---------------------------------------------- device-resident replay target
class DeviceReplayTarget:
    """A replay target kept as a device route table and a row map: token t
    replays ``table[rows[t]]`` (table int32 [N, k], rows int32 [T], both on
    the device).  The router kernels read it directly
    (``ops.router_replay_rows``), so a step's table is uploaded once and a
    micro's row map once for every router, instead of one host-gathered
    [T, k] target per router call (routing_replay.py:1437-1474, 1530-1572)."""

    def __init__(self, table: torch.Tensor, rows: torch.Tensor) -> None:
        if table.dim() != 2 or rows.dim() != 1:
            raise RuntimeError("DeviceReplayTarget needs table [N, k] and rows [T]")
        self.table, self.rows = table, rows

    @property
    def shape(self) -> torch.Size:
        return torch.Size((int(self.rows.shape[0]), int(self.table.shape[1])))

    @property
    def device(self) -> torch.device:
        return self.table.device

    def materialize(self) -> torch.Tensor:
        """The [T, k] int64 target (for consumers that need the ids themselves)."""
        return self.table.index_select(0, self.rows.long()).long()


# ----------------------------------------------------- router replay object
class RouterReplayAction(enum.Enum):
    RECORD = "record"
    REPLAY_FORWARD = "replay_forward"
    REPLAY_BACKWARD = "replay_backward"


class RouterReplay:
    """Per-router replay state with megatron's RouterReplay interface (the
    contract the controller drives, restated from the fake in
    tests/unit/test_moe_routing_replay.py:136-161): a target set with
    ``set_target_indices`` and the REPLAY_FORWARD action replaces top-k."""

    _instances: "weakref.WeakSet[RouterReplay]" = weakref.WeakSet()

    def __init__(self) -> None:
        self.target_topk_idx: torch.Tensor | None = None
        self.recorded_topk_idx: torch.Tensor | None = None
        self.router_replay_action: RouterReplayAction | None = None
        RouterReplay._instances.add(self)

    # class-wide controls
    @staticmethod
    def clear_global_indices() -> None:
        for r in list(RouterReplay._instances):
            r.clear_indices()

    @staticmethod
    def set_global_router_replay_action(action: RouterReplayAction) -> None:
        for r in list(RouterReplay._instances):
            r.router_replay_action = action

    @staticmethod
    def clear_global_router_replay_action() -> None:
        for r in list(RouterReplay._instances):
            r.router_replay_action = None

    # per instance
    def set_target_indices(self, topk_indices: torch.Tensor) -> None:
        self.target_topk_idx = topk_indices

    def set_router_replay_action(self, action: RouterReplayAction | None) -> None:
        self.router_replay_action = action

    def clear_router_replay_action(self) -> None:
        self.router_replay_action = None

    def clear_indices(self) -> None:
        self.target_topk_idx = None
        self.recorded_topk_idx = None

    def record_indices(self, topk_indices: torch.Tensor) -> None:
        self.recorded_topk_idx = topk_indices.detach()

    def get_recorded_indices(self) -> torch.Tensor | None:
        return self.recorded_topk_idx

    def active_target(self) -> torch.Tensor | None:
        """The target that replaces top-k now, or None."""
        if self.router_replay_action == RouterReplayAction.REPLAY_FORWARD:
            return self.target_topk_idx
        return None

    def get_replay_topk(self, scores: torch.Tensor, topk: int, num_groups: int | None = None,
                        group_topk: int | None = None,
                        default_compute_topk: Callable[..., Any] | None = None):
        """(selected scores, indices): the target's scores under REPLAY_FORWARD,
        else the default top-k (recorded under RECORD)."""
        target = self.active_target()
        if target is not None:
            if isinstance(target, DeviceReplayTarget):
                target = target.materialize()
            ids = target.to(device=scores.device, dtype=torch.long)
            return scores.gather(1, ids), ids
        vals, ids = default_compute_topk(scores, topk, num_groups, group_topk)
        if self.router_replay_action == RouterReplayAction.RECORD:
            self.record_indices(ids)
        return vals, ids


# ------------------------------------------------------- parallel topology
class SingleProcessParallelState:
    """The parallel_state the controller consults, for one process on one GPU."""

    def get_tensor_model_parallel_world_size(self) -> int:
        return 1

    def get_tensor_model_parallel_rank(self) -> int:
        return 0

    def get_context_parallel_world_size(self) -> int:
        return 1

    def get_data_parallel_world_size(self) -> int:
        return 1

    def get_data_parallel_rank(self) -> int:
        return 0


class TopologyAwareLocalTokenIndexer:
    """Local token uid order of this rank: context-parallel slice, then the
    sequence-parallel slice of merged rows (routing_replay.py:624-683)."""

    def __init__(self, parallel_state_module: Any | None = None) -> None:
        self._ps = parallel_state_module or SingleProcessParallelState()

    def build_local_token_uids(self, *, global_token_uids: torch.Tensor, num_local_tokens: int,
                               sequence_parallel: bool, context_parallel_size: int) -> torch.Tensor:
        uids = global_token_uids.to(dtype=torch.int64, device="cpu").reshape(-1)
        if context_parallel_size > 1 and int(self._ps.get_context_parallel_world_size()) > 1:
            raise RuntimeError("context-parallel token slicing needs megatron's "
                               "get_batch_on_this_cp_rank, which this build does not provide")
        tp = int(self._ps.get_tensor_model_parallel_world_size())
        if sequence_parallel and tp > 1 and uids.numel() != num_local_tokens:
            total = int(uids.numel())
            if total % tp:
                raise RuntimeError(
                    "Routing replay cannot derive sequence-parallel local token uids from merged "
                    f"rows: total_tokens={total}, tp_size={tp}, num_local_tokens={num_local_tokens}")
            per = total // tp
            if per != num_local_tokens:
                raise RuntimeError(
                    "Routing replay local token uid count mismatch after context-parallel "
                    f"slicing: total_tokens={total}, tp_size={tp}, "
                    f"expected_local_tokens={num_local_tokens}, tp_local_tokens={per}")
            rank = int(self._ps.get_tensor_model_parallel_rank())
            uids = uids[rank * per:(rank + 1) * per]
        uids = uids.contiguous()
        if uids.numel() != num_local_tokens:
            raise RuntimeError("Routing replay local token uid count mismatch: "
                               f"expected={num_local_tokens}, got={uids.numel()}")
        return uids


# ---------------------------------------------------------------- controller
@dataclass
class _RouterCursor:
    """Per-router progress through the step's call sequence."""
    sequence: list[int]
    pos: int = 0
    last_index: int | None = None
    last_key: tuple[str, int] | None = None
    reuses: int = 0


@dataclass
class _Binding:
    module: Any
    original_routing: Any
    router_replay: Any
    sequence_parallel: bool
    context_parallel_size: int
    topk: int


class MoeRoutingReplayController:
    """Feeds each patched router the replay target of the current micro-batch
    (routing_replay.py:696-1579).

    Life cycle per step: ``set_step`` -> for each micro ``begin_micro`` ->
    ``set_local_input_token_uids`` / ``prepare_micro_targets`` (targets are
    built on the host and staged to the device on a side stream, or, with
    ``device_targets``, kept as the step's device route table plus the
    micro's device row map) -> the
    router's ``routing`` call installs the target -> ``finalize_step`` checks
    every expected call was consumed.  A second routing call for the same
    micro (activation recompute) reuses the previous call's route.
    """

    def __init__(self, *, bundle: MoeRoutingReplayBundle, strict: bool,
                 local_token_indexer: Any | None = None, allow_recompute_reuse: bool = True,
                 device: torch.device | str | None = None,
                 parallel_state: Any | None = None, device_targets: bool = False) -> None:
        self.bundle = bundle
        self.strict = strict
        self.allow_recompute_reuse = allow_recompute_reuse
        # device path: route tables uploaded once per step and row maps once
        # per micro; routers replay table[rows[t]] (DeviceReplayTarget)
        self.device_targets = device_targets
        self.parallel_state = parallel_state or SingleProcessParallelState()
        self.local_token_indexer = local_token_indexer or TopologyAwareLocalTokenIndexer(
            self.parallel_state)
        self._device = torch.device(device) if device is not None else None
        self._bindings: dict[str, _Binding] = {}
        self._target_buffers: dict[tuple[str, str, int], torch.Tensor] = {}
        self._copy_stream: torch.cuda.Stream | None = None
        self._reset_step_state()

    # ------------------------------------------------------------ state
    def _reset_step_state(self) -> None:
        self._step: int | None = None
        self._step_routes: StepRoutes | None = None
        self._sample: int | None = None
        self._micro: int | None = None
        self._cursors: dict[str, _RouterCursor] = {}
        self._uid_dense_start: int | None = None
        self._uid_count = 0
        self._uid_rows: dict[int, int] = {}
        if getattr(self, "_device_tables", None) and self._copy_stream is not None:
            # the dropped tables' memory returns to the compute stream: order it after their copies
            torch.cuda.current_stream(self._target_device()).wait_stream(self._copy_stream)
        self._device_tables: dict[tuple[str, int], torch.Tensor] = {}
        self._reset_staged()

    def _reset_staged(self) -> None:
        self._uid_sets: dict[str, torch.Tensor] = {}
        self._targets: dict[tuple[str, str, int], torch.Tensor] = {}
        self._installed: dict[str, tuple[str, int]] = {}
        self._host_staging: list[torch.Tensor] = []
        self._device_rows: dict[tuple[str, bool], torch.Tensor] = {}
        self._copy_event: torch.cuda.Event | None = None
        self._copy_waited = True
        self._active_uid_key: str | None = None

    @property
    def _local_router_keys(self) -> list[str]:
        return sorted(self._bindings)

    def update_bundle(self, *, bundle: MoeRoutingReplayBundle, strict: bool) -> None:
        self.bundle = bundle
        self.strict = strict
        self.clear_replay_state()
        if strict:
            missing = [k for k in self._local_router_keys if k not in bundle.router_keys]
            if missing:
                raise RuntimeError(
                    f"Router keys from model are missing in replay bundle: router_keys={missing}")

    def clear_replay_state(self) -> None:
        self._clear_replay_objects()
        self._reset_step_state()

    def _clear_replay_objects(self) -> None:
        RouterReplay.clear_global_indices()
        RouterReplay.clear_global_router_replay_action()
        for b in self._bindings.values():
            if not isinstance(b.router_replay, RouterReplay):
                b.router_replay.set_router_replay_action(None)

    def _target_device(self) -> torch.device:
        if self._device is not None:
            return self._device
        if torch.cuda.is_available():
            return torch.device("cuda", torch.cuda.current_device())
        return torch.device("cpu")

    # --------------------------------------------------------- patching
    def install_router_patches(self, model_chunks: list[Any]) -> None:
        """Wrap ``routing`` of every ``*.mlp.router`` module so that the replay
        target of the active micro is installed right before it runs."""
        global _active_controller
        if self._bindings:
            return
        for chunk_index, chunk in enumerate(model_chunks):
            for name, module in chunk.named_modules():
                if ROUTER_NAME_TOKEN not in name or not hasattr(module, "routing"):
                    continue
                rk = build_router_key_from_module_name(chunk_index=chunk_index, module_name=name)
                if self.strict and rk not in self.bundle.router_keys:
                    raise RuntimeError(
                        f"Router key from model is missing in replay bundle: router_key='{rk}'")
                config = getattr(module, "config", None)
                if bool(getattr(config, "moe_router_fusion", False)):
                    raise RuntimeError(
                        "MoE routing replay requires moe_router_fusion=False because Megatron "
                        f"Core fused routing bypasses RouterReplay: router_key='{rk}'")
                replay = getattr(module, "router_replay", None)
                if replay is None:
                    raise RuntimeError(
                        "MoE routing replay requires provider.moe_enable_routing_replay=True "
                        f"before model construction: router_key='{rk}'")
                if getattr(replay, "_art_routing_replay_patched", False):
                    raise RuntimeError(f"RouterReplay instance is already patched: router_key='{rk}'")
                if getattr(module, "_art_routing_replay_target_patched", False):
                    raise RuntimeError(
                        f"Router module routing method is already patched: router_key='{rk}'")
                original = module.routing
                install = torch.compiler.disable(
                    lambda _rk=rk: self._prepare_native_target_for_router(_rk))

                def routing_with_replay_target(_module, *args, _orig=original, _install=install,
                                               **kwargs):
                    _install()
                    return _orig(*args, **kwargs)

                module.routing = types.MethodType(routing_with_replay_target, module)
                module._art_routing_replay_target_patched = True
                self._bindings[rk] = _Binding(
                    module=module, original_routing=original, router_replay=replay,
                    sequence_parallel=bool(getattr(config, "sequence_parallel", False)),
                    context_parallel_size=int(getattr(config, "context_parallel_size", 1)),
                    topk=int(module.topk))
        _active_controller = self

    def remove_router_patches(self) -> None:
        global _active_controller
        if _active_controller is self:
            _active_controller = None
        for b in self._bindings.values():
            b.module.routing = b.original_routing
            if hasattr(b.module, "_art_routing_replay_target_patched"):
                delattr(b.module, "_art_routing_replay_target_patched")
        self._clear_replay_objects()
        self._bindings.clear()
        self._target_buffers.clear()
        self._reset_step_state()

    # ------------------------------------------------------------ steps
    def set_step(self, *, step_index: int, sample_index: int | list[int | None] | None,
                 global_grad_accumulation_sequences: int | None = None) -> None:
        if step_index not in self.bundle.steps:
            raise RuntimeError(f"Replay bundle missing step_index={step_index}. "
                               f"Available steps={sorted(self.bundle.steps)}")
        sr = self.bundle.steps[step_index]
        self._reset_step_state()
        self._step, self._step_routes = step_index, sr
        if isinstance(sample_index, list):
            self._sample = next((s for s in sample_index if s is not None), None)
        else:
            self._sample = sample_index
        uids = sr.global_token_uids
        self._uid_count = int(uids.numel())
        self._uid_dense_start = self._dense_start(uids)
        if self._uid_dense_start is None:
            self._uid_rows = {int(u): row for row, u in enumerate(uids.tolist())}
        for rk in self._local_router_keys:
            if rk not in sr.routers:
                raise RuntimeError("Replay bundle step is missing local router key: "
                                   f"step={step_index}, router='{rk}'")
            topk = self._bindings[rk].topk
            for ci, route in sr.routers[rk].calls.items():
                if not bool(route.expert_mask.all()):
                    raise RuntimeError("masked slots are unsupported by Megatron native MoE routing "
                                       f"replay: step={step_index}, router='{rk}', call={ci}")
                if route.max_topk != topk:
                    raise RuntimeError(
                        "Replay route topk does not match Megatron router topk: "
                        f"step={step_index}, router='{rk}', call={ci}, "
                        f"route_topk={route.max_topk}, router_topk={topk}")
            self._cursors[rk] = _RouterCursor(self._call_sequence(
                rk, sample_index, global_grad_accumulation_sequences))
        RouterReplay.clear_global_indices()
        RouterReplay.set_global_router_replay_action(RouterReplayAction.REPLAY_FORWARD)

    def finalize_step(self) -> None:
        if self._step_routes is None:
            raise RuntimeError("finalize_step called before set_step")
        for rk in self._local_router_keys:
            cur = self._cursors.get(rk)
            if cur is None:
                raise RuntimeError("Routing replay call sequence missing for router key: "
                                   f"step={self._step}, router='{rk}'")
            if cur.pos != len(cur.sequence):
                raise RuntimeError("Routing replay step consumption mismatch: "
                                   f"step={self._step}, router='{rk}', consumed={cur.pos}, "
                                   f"expected={len(cur.sequence)}")
        reuses = {rk: c.reuses for rk, c in sorted(self._cursors.items()) if c.reuses}
        if reuses:
            logger.info("Routing replay reused routes for recompute: step=%s counts=%s",
                        self._step, reuses)
        self._clear_replay_objects()
        self._reset_step_state()

    @staticmethod
    def _dense_start(uids: torch.Tensor) -> int | None:
        """First uid when the uids are consecutive (row = uid - start), else None."""
        n = int(uids.numel())
        if n == 0:
            return None
        if n == 1 or bool((uids[1:] - uids[:-1] == 1).all()):
            return int(uids[0])
        return None

    # ------------------------------------------------- call bookkeeping
    def _dummy_key(self, local_micro_index: int) -> tuple[str, int]:
        ps = self.parallel_state
        return ("dummy_micro_slot", local_micro_index * int(ps.get_data_parallel_world_size())
                + int(ps.get_data_parallel_rank()))

    def _micro_key(self, sample: int | None, local_micro_index: int) -> tuple[str, int]:
        return ("sample", int(sample)) if sample is not None else self._dummy_key(local_micro_index)

    def _active_key(self) -> tuple[str, int] | None:
        return None if self._micro is None else self._micro_key(self._sample, self._micro)

    def _call_sequence(self, rk: str, sample_index, gga: int | None) -> list[int]:
        """Order in which this rank consumes the step's calls of router ``rk``."""
        calls = self._step_routes.routers[rk].calls
        if all(r.call_key is not None for r in calls.values()):
            by_key: dict[tuple[str, int], list[int]] = defaultdict(list)
            for ci in sorted(calls):
                by_key[calls[ci].call_key].append(ci)
            if isinstance(sample_index, list):
                local_keys = [self._micro_key(s, i) for i, s in enumerate(sample_index)]
            else:
                local_keys = [self._micro_key(sample_index, 0)]
            seq: list[int] = []
            for key in local_keys:
                if not by_key.get(key):
                    raise RuntimeError("Replay router call sequence is missing local micro metadata: "
                                       f"step={self._step}, router='{rk}', call_key={key}")
                seq.extend(by_key[key])
            return seq
        # calls without micro metadata: contiguous blocks of calls per sample
        total = len(calls)
        if sample_index is None:
            if total != 1:
                raise RuntimeError(f"Replay router call sequence lacks sample metadata and has "
                                   f"{total} calls for router='{rk}', step={self._step}")
            return [0]
        samples = [s for s in sample_index if s is not None] if isinstance(sample_index, list) \
            else [sample_index]
        per_step = gga if gga is not None else len(samples)
        if per_step <= 0 or total % per_step:
            raise RuntimeError("Replay router call count is not divisible by step sample count: "
                               f"step={self._step}, router='{rk}', total_calls={total}, "
                               f"step_sample_count={per_step}")
        per_sample = total // per_step
        base = self._step * per_step
        seq = []
        for s in samples:
            off = int(s) - base
            if not 0 <= off < per_step:
                raise RuntimeError("Replay router call index is outside the step-local range: "
                                   f"step={self._step}, router='{rk}', sample_index={s}, "
                                   f"step_base_sample_index={base}, step_sample_count={per_step}")
            seq.extend(range(off * per_sample, (off + 1) * per_sample))
        return seq

    def _active_calls(self, rk: str) -> list[int]:
        """Calls of router ``rk`` that belong to the active micro (the previous
        call again when the micro re-runs its forward)."""
        if self._step_routes is None:
            raise RuntimeError("Routing replay begin_micro called before set_step")
        calls = self._step_routes.routers[rk].calls
        cur = self._cursors[rk]
        key = self._active_key()
        repeat = key is not None and cur.last_index is not None and cur.last_key == key
        if cur.pos >= len(cur.sequence):
            return [cur.last_index] if repeat else []
        if key is None:
            return [cur.sequence[cur.pos]]
        if repeat and calls[cur.sequence[cur.pos]].call_key != key:
            return [cur.last_index]
        run = []
        for ci in cur.sequence[cur.pos:]:
            if calls[ci].call_key != key:
                break
            run.append(ci)
        return run

    def _next_call(self, rk: str) -> int:
        """Consume (or, for a recompute, reuse) the next call of router ``rk``."""
        if self._step_routes is None:
            raise RuntimeError("Routing replay router call occurred before set_step")
        cur = self._cursors.get(rk)
        if cur is None:
            raise RuntimeError("Routing replay call sequence missing for router key: "
                               f"step={self._step}, router='{rk}'")
        calls = self._step_routes.routers[rk].calls
        key = self._active_key()
        nxt = calls[cur.sequence[cur.pos]].call_key if cur.pos < len(cur.sequence) else None
        if key is not None and cur.last_index is not None and cur.last_key == key and nxt != key:
            if not self.allow_recompute_reuse:
                raise RuntimeError("Routing replay recompute reuse is disabled: "
                                   f"step={self._step}, router='{rk}', call_key={key}")
            cur.reuses += 1
            return cur.last_index
        if cur.pos >= len(cur.sequence):
            raise RuntimeError("Routing replay call cursor exceeded local call sequence: "
                               f"step={self._step}, router='{rk}', cursor={cur.pos}, "
                               f"sequence_length={len(cur.sequence)}")
        ci = cur.sequence[cur.pos]
        cur.pos += 1
        cur.last_index, cur.last_key = ci, calls[ci].call_key
        return ci

    # ------------------------------------------------------------ micros
    def begin_micro(self, sample_index: int | None, micro_order: int) -> None:
        self._sample, self._micro = sample_index, micro_order
        for rk in self._local_router_keys:
            calls = self._active_calls(rk)
            if len(calls) != 1:
                raise RuntimeError("Routing replay expected exactly one router call per local "
                                   f"microbatch for router='{rk}', got {calls}")

    def set_local_input_token_uids(self, local_token_uids: torch.Tensor | None) -> None:
        self.prepare_micro_targets({"attention": local_token_uids})

    def prepare_micro_targets(self, token_uid_sets: Mapping[str, torch.Tensor | None], *,
                              active_token_uid_key: str = "attention") -> None:
        """Build and stage the targets of every router for each token layout."""
        if self._step_routes is None or self._micro is None:
            raise RuntimeError("Routing replay target staging requires set_step and begin_micro")
        self._reset_staged()
        sets = {k: self._normalize_uids(v) for k, v in token_uid_sets.items() if v is not None}
        if not sets:
            raise RuntimeError("Routing replay requires at least one token UID set")
        if active_token_uid_key not in sets:
            raise RuntimeError("Routing replay active token UID key was not prepared: "
                               f"key='{active_token_uid_key}', prepared={sorted(sets)}")
        self._uid_sets = sets
        if not self._bindings:
            self._active_uid_key = active_token_uid_key
            return
        use_device = self.device_targets and self._target_device().type == "cuda"
        for uk, uids in sets.items():
            for rk in self._local_router_keys:
                calls = self._active_calls(rk)
                if len(calls) != 1:
                    raise RuntimeError("Routing replay expected exactly one active router call while "
                                       f"staging targets for router='{rk}', got {calls}")
                b = self._bindings[rk]
                router_uids = self._token_uids_for_router_binding(
                    uids, sequence_parallel=b.sequence_parallel)
                if use_device and bool((router_uids >= 0).all()):
                    # padded uids (< 0) take synthetic rows: those micros stay on the host path
                    self._stage_device((uk, rk, calls[0]), router_uids, b.sequence_parallel)
                    continue
                target = self._explicit_target_for_router_call(
                    router_key=rk, call_index=calls[0], explicit_uids=router_uids)
                self._stage((uk, rk, calls[0]), target)
        if self._copy_stream is not None and not self._copy_waited:
            self._copy_event = torch.cuda.Event()
            self._copy_event.record(self._copy_stream)
        self.set_active_token_uid_key(active_token_uid_key)

    def set_active_token_uid_key(self, token_uid_key: str) -> None:
        if self._bindings and token_uid_key not in {k[0] for k in self._targets}:
            raise RuntimeError("Routing replay token UID key was not staged for this micro: "
                               f"key='{token_uid_key}', staged={sorted({k[0] for k in self._targets})}")
        self._active_uid_key = token_uid_key

    @staticmethod
    def _normalize_uids(uids: torch.Tensor) -> torch.Tensor:
        if uids.device.type != "cpu":
            raise RuntimeError(
                "Routing replay token UIDs must be CPU metadata. Passing CUDA token UIDs would "
                "force a host/device synchronization in the model path.")
        return uids.detach().to(torch.int64).contiguous().reshape(-1)

    def local_token_uids_for_active_dispatch(self, *, num_local_tokens: int,
                                             sequence_parallel: bool) -> torch.Tensor | None:
        if self._active_uid_key is None:
            return None
        uids = self._uid_sets.get(self._active_uid_key)
        if uids is None:
            return None
        local = self._token_uids_for_router_binding(uids, sequence_parallel=sequence_parallel)
        if local.numel() == num_local_tokens:
            return local.contiguous()
        compact = local[local >= 0]
        return compact.contiguous() if compact.numel() == num_local_tokens else None

    def _token_uids_for_router_binding(self, token_uids: torch.Tensor, *,
                                       sequence_parallel: bool) -> torch.Tensor:
        """This tensor-parallel rank's ceil(N/tp) slice under sequence
        parallelism, padded with uid -1 (routing_replay.py:1506-1528)."""
        if not sequence_parallel:
            return token_uids
        tp = int(self.parallel_state.get_tensor_model_parallel_world_size())
        if tp <= 1:
            return token_uids
        rank = int(self.parallel_state.get_tensor_model_parallel_rank())
        n = int(token_uids.numel())
        per = (n + tp - 1) // tp
        lo, hi = rank * per, min(rank * per + per, n)
        out = token_uids.new_full((per,), -1)
        if lo < n:
            out[:hi - lo] = token_uids[lo:hi]
        return out

    def _explicit_target_for_router_call(self, *, router_key: str, call_index: int,
                                         explicit_uids: torch.Tensor) -> torch.Tensor:
        """[N, k] int64 target: the bundle row of each uid, synthetic rows for
        uid < 0 (routing_replay.py:1437-1474)."""
        if self._step_routes is None:
            raise RuntimeError("Routing replay explicit target used before set_step")
        route = self._step_routes.routers[router_key].calls[call_index]
        uids = explicit_uids.reshape(-1).contiguous()
        target = torch.empty((uids.numel(), route.max_topk), dtype=torch.long)
        ok = torch.nonzero(uids >= 0).reshape(-1)
        if ok.numel():
            rows = self._rows_for_uids(uids[ok], router_key, call_index)
            target[ok] = route.expert_indices.index_select(0, rows).long()
        pad = torch.nonzero(uids < 0).reshape(-1)
        if pad.numel():
            target[pad] = synthetic_replay_rows(
                row_positions=pad, num_experts=route.num_experts, topk=route.max_topk,
                dtype=torch.long,
                seed=(int(self._step or 0) + 1) * _SEED_SAMPLE + (call_index + 1) * _SEED_LAYER)
        return target.contiguous()

    def _rows_for_uids(self, uids: torch.Tensor, rk: str, ci: int) -> torch.Tensor:
        if self._uid_dense_start is not None:
            rows = uids.long() - self._uid_dense_start
            bad = (rows < 0) | (rows >= self._uid_count)
            if bool(bad.any()):
                raise RuntimeError("Explicit routing replay token uid is outside the active dense "
                                   f"step span: step={self._step}, router='{rk}', call={ci}, "
                                   f"uid={int(uids[bad][0])}")
            return rows
        try:
            return torch.tensor([self._uid_rows[u] for u in uids.tolist()], dtype=torch.long)
        except KeyError as exc:
            raise RuntimeError("Explicit routing replay token uid is missing from the active step "
                               f"map: step={self._step}, router='{rk}', call={ci}, "
                               f"uid={exc.args[0]}") from exc

    def _stage(self, key: tuple[str, str, int], target_cpu: torch.Tensor) -> None:
        """Keep the target on the host (CPU device) or start its copy into a
        reused device buffer on a side stream from pinned host memory."""
        target_cpu = target_cpu.long().contiguous()
        dev = self._target_device()
        if dev.type != "cuda":
            self._targets[key] = target_cpu
            return
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=dev)
        host = target_cpu if target_cpu.is_pinned() else target_cpu.pin_memory()
        self._host_staging.append(host)
        buf = self._target_buffers.get(key)
        if buf is None or buf.shape != host.shape or buf.device != dev:
            buf = torch.empty(host.shape, dtype=torch.long, device=dev)
            self._target_buffers[key] = buf
        # the copy must not overwrite a buffer the compute stream may still read
        self._copy_stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self._copy_stream):
            buf.copy_(host, non_blocking=True)
        self._targets[key] = buf
        self._copy_waited = False

    def _copy_to_device(self, host: torch.Tensor) -> torch.Tensor:
        """Start an async copy of ``host`` (pinned) into a new device buffer on
        the side stream; the buffer belongs to the compute stream."""
        dev = self._target_device()
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=dev)
        host = host.contiguous()
        host = host if host.is_pinned() else host.pin_memory()
        self._host_staging.append(host)
        buf = torch.empty(host.shape, dtype=host.dtype, device=dev)
        self._copy_stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self._copy_stream):
            buf.copy_(host, non_blocking=True)
        self._copy_waited = False
        return buf

    def _stage_device(self, key: tuple[str, str, int], uids: torch.Tensor,
                      sequence_parallel: bool) -> None:
        """Device path: the step's route table of the call (uploaded once per
        step) and the micro's row map (uploaded once per token layout)."""
        uk, rk, ci = key
        table = self._device_tables.get((rk, ci))
        if table is None:
            route = self._step_routes.routers[rk].calls[ci]
            table = self._copy_to_device(route.expert_indices.to(torch.int32))
            self._device_tables[(rk, ci)] = table
        rows = self._device_rows.get((uk, sequence_parallel))
        if rows is None:
            rows = self._copy_to_device(self._rows_for_uids(uids, rk, ci).to(torch.int32))
            self._device_rows[(uk, sequence_parallel)] = rows
        self._targets[key] = DeviceReplayTarget(table, rows)

    def wait_for_staged_targets(self) -> None:
        if self._copy_event is None or self._copy_waited:
            return
        torch.cuda.current_stream(self._target_device()).wait_event(self._copy_event)
        self._copy_waited = True

    def _prepare_native_target_for_router(self, router_key: str) -> None:
        """Install the active micro's target on router ``router_key`` (runs
        right before its ``routing``; routing_replay.py:1388-1435)."""
        if self._step_routes is None or self._micro is None or self._active_uid_key is None:
            raise RuntimeError("Routing replay router call occurred before staged targets were "
                               f"ready: router='{router_key}'")
        calls = self._active_calls(router_key)
        if len(calls) != 1:
            raise RuntimeError("Routing replay expected exactly one active router call while "
                               f"preparing native replay for router='{router_key}', got {calls}")
        ci = self._next_call(router_key)
        if ci != calls[0]:
            raise RuntimeError("Routing replay cursor mismatch while preparing native replay: "
                               f"router='{router_key}', expected={calls[0]}, actual={ci}")
        tkey = (self._active_uid_key, ci)
        if self._installed.get(router_key) == tkey:
            return
        self.wait_for_staged_targets()
        target = self._targets.get((self._active_uid_key, router_key, ci))
        if target is None:
            raise RuntimeError("Routing replay target was not staged before router execution: "
                               f"step={self._step}, router='{router_key}', call={ci}, "
                               f"token_uid_key='{self._active_uid_key}'")
        b = self._bindings[router_key]
        if int(target.shape[1]) != b.topk:
            raise RuntimeError("Routing replay target topk mismatch at router call: "
                               f"router='{router_key}', call={ci}, "
                               f"target_topk={int(target.shape[1])}, router_topk={b.topk}")
        b.router_replay.set_target_indices(target)
        b.router_replay.set_router_replay_action(RouterReplayAction.REPLAY_FORWARD)
        self._installed[router_key] = tkey
