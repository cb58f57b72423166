"""MoE routing replay: route bundles, their builder, and the controller that
feeds each router its replayed top-k ids, device-first.

What is kept from the reference (/root/reference/src/art/megatron/routing_replay.py)
because it is format or interface:

* the on-disk bundle ``moe_routing_replay_v2``: ``manifest.json`` plus one
  ``step_%06d.safetensors`` per step holding ``global_token_uids`` and
  ``<router key>/call_<i>/expert_indices|expert_mask[|expert_probs]``
  (:288-462), and router keys ``chunk_CC.layer_LLLL.mlp.router`` (:89-115);
* the public classes and the controller methods a trainer calls
  (``install_router_patches``, ``set_step``, ``begin_micro``,
  ``set_local_input_token_uids`` / ``prepare_micro_targets``,
  ``set_active_token_uid_key``, ``finalize_step``, ...), the megatron
  ``RouterReplay`` driving contract (:1388-1435) and the error fragments the
  reference's tests match (tests/unit/test_moe_routing_replay.py:439-524);
* the synthetic-route seeds: ``random.Random(seed + (pos+1)*1_299_709)
  .sample(range(E), k)`` with seed ``(sample+1)*1_000_003 + (layer+1)*97_003``
  for captured sequences, ``+ (slot+1)*9_176`` with the step in place of the
  sample for padded micro slots, and ``(step+1)*1_000_003 + (call+1)*97_003``
  for tokens staged without a uid (:538-555, 594-610, 1471-1472).

How it works here.  A step's routes are validated once at ``set_step`` and,
on a GPU, every call this rank will consume is copied into ONE device route
table (all routers and calls back to back, a single pinned host-to-device
copy on a side stream).  A micro's token uids are turned into step rows by a
vectorised uid index (dense offset or sorted lookup) once per uid layout;
that int32 row map is uploaded once and shared by every router, and each
router call's target is a view ``(table[call rows], row map)`` that the HIP
replay kernel reads directly (``ops.router_replay_rows``).  Tokens without a
uid (negative uids) get synthetic rows in a small per-call side table that
the row map addresses with negative entries.  On the CPU, or with
``device_targets=False``, targets are plain ``[T, k]`` int64 tensors (what
megatron's own RouterReplay consumes).  Call consumption per router is a
small cursor state machine that also recognises activation-recompute calls.
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
from collections.abc import Iterable, Mapping
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable

import numpy as np
import torch

logger = logging.getLogger(__name__)

ROUTER_NAME_TOKEN = ".mlp.router"
ROUTER_KEY_FORMAT_VERSION = "moe_routing_replay_v2"
GLOBAL_TOKEN_UIDS_KEY = "global_token_uids"

# seed formula of the synthetic routes (a data-format contract)
_SEED_SAMPLE = 1_000_003
_SEED_LAYER = 97_003
_SEED_SLOT = 9_176
_SEED_POSITION = 1_299_709

_LAYER_PATH = re.compile(r"decoder\.layers\.(?P<layer>\d+)\.mlp\.router$")
_TRACE_PREFIX = re.compile(r"^chunk(?P<chunk>\d+)\.(?P<name>.+)$")

_installed: "weakref.ReferenceType[MoeRoutingReplayController] | None" = None


def active_routing_replay_controller() -> "MoeRoutingReplayController | None":
    """The controller whose router patches are currently installed, if any."""
    return _installed() if _installed is not None else None


# ----------------------------------------------------------------- router keys
_DOUBLED = frozenset({"linear_proj", "linear_qkv", "in_proj", "linear_fc1", "linear_fc2"})


def canonical_module_name(name: str) -> str:
    """A module path without wrapper segments: leading ``module.``, every
    ``_orig_mod`` (torch.compile), a fused linear named twice in a row, and
    the LoRA wrappers around an output projection
    (weights/param_name_canonicalization.py:17-54)."""
    out: list[str] = []
    for part in name.split("."):
        if part == "_orig_mod" or (part == "module" and not out):
            continue
        prev = out[-1] if out else None
        if part in _DOUBLED and prev == part:
            continue                        # linear_fc1.linear_fc1 -> linear_fc1
        if part == "linear_proj" and prev == "out_proj":
            continue                        # out_proj.linear_proj -> out_proj
        if part == "linear_proj" and prev == "row_parallel_lora":
            out.pop()                       # row_parallel_lora.linear_proj -> (nothing)
            continue
        out.append(part)
    return ".".join(out)


def build_router_key_from_module_name(*, chunk_index: int, module_name: str) -> str:
    """``chunk_CC.layer_LLLL.mlp.router`` of a router module path."""
    clean = canonical_module_name(module_name)
    found = _LAYER_PATH.search(clean)
    if found is None:
        raise RuntimeError(f"Unable to derive router key from module name '{module_name}' "
                           f"(as '{clean}'): it must end in 'decoder.layers.<n>.mlp.router'")
    return f"chunk_{chunk_index:02d}.layer_{int(found['layer']):04d}.mlp.router"


def build_router_key_from_trace_name(trace_module_name: str) -> str:
    """Router key of a forward-trace name ``chunk<idx>.<module path>``."""
    found = _TRACE_PREFIX.match(trace_module_name)
    if found is None:
        raise RuntimeError(f"trace name '{trace_module_name}' does not start with 'chunk<idx>.'")
    return build_router_key_from_module_name(chunk_index=int(found["chunk"]),
                                             module_name=found["name"])


# ---------------------------------------------------------------- bundle types
def _host(t: Any, dtype: torch.dtype, what: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what} must be a torch.Tensor, got {type(t).__name__}")
    return t.detach().to(device="cpu", dtype=dtype).contiguous()


@dataclass
class ParallelTopology:
    """Parallel layout the routes were captured under (manifest ``topology``)."""
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
        return cls(**{k: (bool(v) if k == "sp" else int(v)) for k, v in d.items()})


def parallel_topology_from_env() -> ParallelTopology:
    """The topology the ART_MEGATRON_* environment describes (one process)."""
    def num(*names: str) -> int:
        for n in names:
            v = os.environ.get(n)
            if v:
                return int(v)
        return 1
    tp = num("ART_MEGATRON_TENSOR_MODEL_PARALLEL_SIZE")
    return ParallelTopology(
        tp=tp, ep=num("ART_MEGATRON_EXPERT_MODEL_PARALLEL_SIZE"),
        etp=num("ART_MEGATRON_EXPERT_TENSOR_PARALLEL_SIZE",
                "ART_MEGATRON_EXPERT_TENSOR_MODEL_PARALLEL_SIZE"),
        dp=1, sp=tp > 1, cp=num("ART_MEGATRON_CONTEXT_PARALLEL_SIZE"),
        pp=num("ART_MEGATRON_PIPELINE_MODEL_PARALLEL_SIZE"))


@dataclass
class RouterCallRoute:
    """Captured top-k ids of one router call: ``expert_indices`` int32
    [tokens, k] (every slot valid: ``expert_mask`` all true), optional
    ``expert_probs``; ``sample_index`` / ``micro_slot`` say which micro it
    belongs to (neither: the legacy call-order layout).  ``expert_indices``
    may live on a GPU (a view of a step's device route table, see
    ``MoeRoutingReplayBundle.from_dir(device=...)``): its id range is then
    checked where it was staged, not here."""
    expert_indices: torch.Tensor
    expert_mask: torch.Tensor
    num_experts: int
    expert_probs: torch.Tensor | None = None
    sample_index: int | None = None
    micro_slot: int | None = None
    rank_token_counts: tuple[int, ...] | None = None

    def __post_init__(self) -> None:
        on_device = isinstance(self.expert_indices, torch.Tensor) and \
            self.expert_indices.device.type != "cpu"
        if on_device:
            if self.expert_indices.dtype != torch.int32 or not self.expert_indices.is_contiguous():
                raise RuntimeError("device expert_indices must be contiguous int32")
        else:
            self.expert_indices = _host(self.expert_indices, torch.int32, "expert_indices")
        self.expert_mask = _host(self.expert_mask, torch.bool, "expert_mask")
        if self.expert_probs is not None:
            self.expert_probs = _host(self.expert_probs, torch.float32, "expert_probs")
        shape = tuple(self.expert_indices.shape)
        if len(shape) != 2:
            raise RuntimeError(f"expert_indices is [tokens, topk], got shape {shape}")
        for name, t in (("expert_mask", self.expert_mask), ("expert_probs", self.expert_probs)):
            if t is not None and tuple(t.shape) != shape:
                raise RuntimeError(f"{name} has shape {tuple(t.shape)}, expert_indices {shape}")
        if not bool(self.expert_mask.all()):
            raise RuntimeError("masked slots are unsupported by native MoE routing replay: every "
                               "replayed token needs a full row of top-k expert ids")
        self.num_experts = int(self.num_experts)
        if self.num_experts <= 0:
            raise RuntimeError(f"num_experts must be positive, got {self.num_experts}")
        if not on_device and self.expert_indices.numel() and (
                int(self.expert_indices.min()) < 0 or
                int(self.expert_indices.max()) >= self.num_experts):
            raise RuntimeError(f"expert_indices hold ids outside [0, {self.num_experts})")
        if self.sample_index is not None:
            self.sample_index = int(self.sample_index)
        if self.micro_slot is not None:
            self.micro_slot = int(self.micro_slot)
        if self.rank_token_counts is not None:
            counts = tuple(int(c) for c in self.rank_token_counts)
            if min(counts, default=0) < 0 or sum(counts) != shape[0]:
                raise RuntimeError(f"rank_token_counts {counts} must be non-negative and sum to "
                                   f"the {shape[0]} route tokens")
            self.rank_token_counts = counts

    @property
    def num_global_tokens(self) -> int:
        return int(self.expert_indices.shape[0])

    @property
    def max_topk(self) -> int:
        return int(self.expert_indices.shape[1])

    @property
    def call_key(self) -> tuple[str, int] | None:
        """Which micro the call belongs to: ("sample", i), ("dummy_micro_slot", j) or None."""
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
            raise RuntimeError("a router needs at least one call per step")
        if min(self.calls) < 0:
            raise RuntimeError(f"call indices must be >= 0, got {sorted(self.calls)}")


@dataclass
class StepRoutes:
    routers: dict[str, StepRouterRoutes]
    global_token_uids: torch.Tensor

    def __post_init__(self) -> None:
        if not self.routers:
            raise RuntimeError("a step needs at least one router")
        uids = _host(self.global_token_uids, torch.int64, "global_token_uids")
        if uids.dim() != 1:
            raise RuntimeError(f"global_token_uids is [tokens], got shape {tuple(uids.shape)}")
        if torch.unique(uids).numel() != uids.numel():
            raise RuntimeError("global_token_uids must be unique per step")
        self.global_token_uids = uids
        n = uids.numel()
        per_micro: dict[tuple[str, int], int] = {}
        for rk, rr in self.routers.items():
            for ci, route in rr.calls.items():
                key, rows = route.call_key, route.num_global_tokens
                if key is None and rows != n:
                    raise RuntimeError(f"router '{rk}' call {ci}: {rows} route rows must match step "
                                       f"global_token_uids ({n}) without per-micro metadata")
                if key is None:
                    continue
                if rows > n:
                    raise RuntimeError(f"router '{rk}' call {ci}: {rows} route rows exceed the "
                                       f"step's {n} global_token_uids")
                if per_micro.setdefault(key, rows) != rows:
                    raise RuntimeError(f"router '{rk}' call {ci}: micro {key} has {rows} route "
                                       f"rows here and {per_micro[key]} elsewhere")


def _tensor_key(router_key: str, call_index: int, name: str) -> str:
    return f"{router_key}/call_{call_index}/{name}"


@dataclass
class MoeRoutingReplayBundle:
    topology: ParallelTopology
    num_steps: int
    max_topk: int
    router_keys: list[str]
    steps: dict[int, StepRoutes]
    format_version: str = ROUTER_KEY_FORMAT_VERSION

    def __post_init__(self) -> None:
        if self.format_version != ROUTER_KEY_FORMAT_VERSION:
            raise RuntimeError(f"bundle format {self.format_version!r} is not "
                               f"{ROUTER_KEY_FORMAT_VERSION!r}")
        if self.num_steps <= 0 or self.max_topk <= 0:
            raise RuntimeError(f"num_steps ({self.num_steps}) and max_topk ({self.max_topk}) "
                               "must be positive")
        keys = list(self.router_keys)
        if not keys or len(set(keys)) != len(keys):
            raise RuntimeError(f"router_keys must be non-empty and unique, got {keys}")
        if set(self.steps) != set(range(self.num_steps)):
            raise RuntimeError(f"steps must contain exactly 0..{self.num_steps - 1}, "
                               f"got {sorted(self.steps)}")
        for si, step in self.steps.items():
            if set(step.routers) != set(keys):
                raise RuntimeError(f"step {si} has routers {sorted(step.routers)}, the bundle "
                                   f"{sorted(keys)}")
            for rr in step.routers.values():
                for route in rr.calls.values():
                    if route.max_topk > self.max_topk:
                        raise RuntimeError(f"a route's topk {route.max_topk} exceeds bundle "
                                           f"max_topk {self.max_topk}")

    # -------------------------------------------------------------- on disk
    def to_dir(self, bundle_dir: str | Path) -> None:
        from safetensors.torch import save_file
        base = Path(bundle_dir)
        base.mkdir(parents=True, exist_ok=True)
        steps_manifest: dict[str, Any] = {}
        for si in sorted(self.steps):
            step = self.steps[si]
            tensors = {GLOBAL_TOKEN_UIDS_KEY: step.global_token_uids}
            routers: dict[str, Any] = {}
            for rk in sorted(step.routers):
                calls: dict[str, Any] = {}
                for ci in sorted(step.routers[rk].calls):
                    route = step.routers[rk].calls[ci]
                    tensors[_tensor_key(rk, ci, "expert_indices")] = route.expert_indices.cpu()
                    tensors[_tensor_key(rk, ci, "expert_mask")] = route.expert_mask
                    if route.expert_probs is not None:
                        tensors[_tensor_key(rk, ci, "expert_probs")] = route.expert_probs
                    info: dict[str, Any] = {"num_experts": route.num_experts}
                    for name in ("sample_index", "micro_slot"):
                        if getattr(route, name) is not None:
                            info[name] = getattr(route, name)
                    if route.rank_token_counts is not None:
                        info["rank_token_counts"] = list(route.rank_token_counts)
                    calls[str(ci)] = info
                routers[rk] = calls
            fname = f"step_{si:06d}.safetensors"
            save_file(tensors, str(base / fname))
            steps_manifest[str(si)] = {"file": fname, "routers": routers}
        manifest = {"format_version": self.format_version, "topology": self.topology.to_json(),
                    "num_steps": self.num_steps, "max_topk": self.max_topk,
                    "router_keys": list(self.router_keys), "steps": steps_manifest}
        (base / "manifest.json").write_text(json.dumps(manifest, indent=2, sort_keys=True),
                                            encoding="utf-8")

    @classmethod
    def from_dir(cls, bundle_dir: str | Path, *,
                 device: torch.device | str | None = None) -> "MoeRoutingReplayBundle":
        """Load a bundle.  With a GPU ``device``, each step's expert ids go
        from the file straight into one device route table per step (all
        routers and calls back to back: read into pinned memory, range-checked
        there, one host-to-device copy); masks, probabilities and token uids
        stay host metadata."""
        from safetensors.torch import load_file
        dev = torch.device(device) if device is not None else None
        if dev is not None and dev.type == "cpu":
            dev = None
        base = Path(bundle_dir)
        mpath = base / "manifest.json"
        if not mpath.exists():
            raise FileNotFoundError(f"no routing replay manifest at {mpath}")
        manifest = json.loads(mpath.read_text(encoding="utf-8"))
        if manifest.get("format_version") != ROUTER_KEY_FORMAT_VERSION:
            raise RuntimeError(f"bundle format {manifest.get('format_version')!r} is not "
                               f"{ROUTER_KEY_FORMAT_VERSION!r}")
        steps: dict[int, StepRoutes] = {}
        for si, sinfo in manifest["steps"].items():
            # clone: the loaded tensors may map the file, which must not stay
            # open (shared-filesystem cleanup) while a long-lived rank holds them
            if dev is None:
                raw = {k: v.clone() for k, v in load_file(str(base / sinfo["file"])).items()}
            else:
                raw = _load_step_to_device(base / sinfo["file"], sinfo["routers"], dev)
            if GLOBAL_TOKEN_UIDS_KEY not in raw:
                raise RuntimeError(f"{sinfo['file']} lacks '{GLOBAL_TOKEN_UIDS_KEY}'")
            routers: dict[str, StepRouterRoutes] = {}
            for rk, cinfo in sinfo["routers"].items():
                calls: dict[int, RouterCallRoute] = {}
                for ci_s, info in cinfo.items():
                    ci = int(ci_s)
                    need = [_tensor_key(rk, ci, n) for n in ("expert_indices", "expert_mask")]
                    absent = [k for k in need if k not in raw]
                    if absent:
                        raise RuntimeError(f"{sinfo['file']} lacks {absent}")
                    calls[ci] = RouterCallRoute(
                        expert_indices=raw[need[0]], expert_mask=raw[need[1]],
                        expert_probs=raw.get(_tensor_key(rk, ci, "expert_probs")),
                        num_experts=int(info["num_experts"]), sample_index=info.get("sample_index"),
                        micro_slot=info.get("micro_slot"),
                        rank_token_counts=info.get("rank_token_counts"))
                routers[rk] = StepRouterRoutes(calls=calls)
            steps[int(si)] = StepRoutes(routers=routers, global_token_uids=raw[GLOBAL_TOKEN_UIDS_KEY])
        return cls(topology=ParallelTopology.from_json(manifest["topology"]),
                   num_steps=int(manifest["num_steps"]), max_topk=int(manifest["max_topk"]),
                   router_keys=list(manifest["router_keys"]), steps=steps,
                   format_version=manifest["format_version"])


_SAFETENSORS_INT = {"I8": np.int8, "I16": np.int16, "I32": np.int32, "I64": np.int64,
                    "U8": np.uint8, "U16": np.uint16, "U32": np.uint32, "U64": np.uint64}


def _load_step_to_device(path: Path, routers: Mapping[str, Any],
                         dev: torch.device) -> dict[str, torch.Tensor]:
    """One step file: every ``expert_indices`` tensor read from the file into
    one pinned int32 buffer (in router, call order), its ids checked against
    the call's ``num_experts``, then one copy into a device table whose views
    are returned; every other tensor is loaded on the host.  The file layout
    is the safetensors one: an 8-byte little-endian header length, a JSON
    header of {name: {dtype, shape, data_offsets}}, then the data."""
    from safetensors import safe_open
    with open(path, "rb") as fh:
        hlen = int.from_bytes(fh.read(8), "little")
        header = json.loads(fh.read(hlen))
        data0 = 8 + hlen
        ids = []
        for rk in sorted(routers):
            for ci in sorted(routers[rk], key=int):
                name = _tensor_key(rk, int(ci), "expert_indices")
                if name not in header:
                    raise RuntimeError(f"{path.name} lacks ['{name}']")
                info = header[name]
                if info["dtype"] not in _SAFETENSORS_INT or len(info["shape"]) != 2:
                    raise RuntimeError(f"{path.name}: {name} must be a 2-D integer tensor, got "
                                       f"{info['dtype']} {info['shape']}")
                ids.append((name, info, int(routers[rk][ci]["num_experts"])))
        total = sum(int(np.prod(i["shape"])) for _, i, _ in ids)
        pinned = torch.empty(total, dtype=torch.int32, pin_memory=True)
        host = pinned.numpy()
        views: list[tuple[str, int, tuple[int, int]]] = []
        at = 0
        for name, info, n_exp in ids:
            b, e = (int(x) for x in info["data_offsets"])
            shape = tuple(int(x) for x in info["shape"])
            n = shape[0] * shape[1]
            fh.seek(data0 + b)
            dt = np.dtype(_SAFETENSORS_INT[info["dtype"]]).newbyteorder("<")
            if e - b != n * dt.itemsize:
                raise RuntimeError(f"{path.name}: {name} byte range does not match its shape")
            if dt == np.dtype("<i4"):
                fh.readinto(memoryview(host[at:at + n]).cast("B"))
            else:
                host[at:at + n] = np.frombuffer(fh.read(e - b), dtype=dt)
            part = host[at:at + n]
            if n and (int(part.min()) < 0 or int(part.max()) >= n_exp):
                raise RuntimeError(f"expert_indices hold ids outside [0, {n_exp})")
            views.append((name, at, shape))
            at += n
    table = torch.empty(total, dtype=torch.int32, device=dev)
    table.copy_(pinned, non_blocking=True)
    torch.cuda.current_stream(dev).synchronize()     # the pinned buffer is released below
    raw = {name: table[a:a + sh[0] * sh[1]].view(sh) for name, a, sh in views}
    with safe_open(str(path), framework="pt") as f:
        for name in f.keys():
            if name not in raw:
                raw[name] = f.get_tensor(name).clone()
    return raw


# ---------------------------------------------------------- synthetic routes
def synthetic_replay_rows(*, row_positions: torch.Tensor | Iterable[int], num_experts: int,
                          topk: int, dtype: torch.dtype, seed: int) -> torch.Tensor:
    """[len(positions), topk] distinct expert ids per position from Python's
    ``random.Random(seed + (position + 1) * 1_299_709).sample(range(E), k)``:
    routes for tokens that have none, reproducible from (seed, position)."""
    positions = row_positions.tolist() if isinstance(row_positions, torch.Tensor) \
        else list(row_positions)
    experts = range(num_experts)
    out = torch.empty((len(positions), topk), dtype=dtype)
    for i, pos in enumerate(positions):
        out[i] = torch.tensor(random.Random(seed + (int(pos) + 1) * _SEED_POSITION)
                              .sample(experts, topk), dtype=dtype)
    return out


# ------------------------------------------------------------------- builder
def _route_free_rows(group_ids: torch.Tensor, parent_ids: torch.Tensor,
                     logprobs: torch.Tensor) -> torch.Tensor:
    """Rows whose missing route cannot matter, [S, seq] bool: terminal
    completion tokens (a branch row whose next row starts another group) and
    branch rows after which no token of the same group is scored (vLLM ran
    no forward for a sequence's last token; prefix-tree packing may leave a
    masked suffix in the branch).  The second set is found in one pass: a
    row p of group g is free if g's last scored row is not after p."""
    real = group_ids != -1
    branch = real & (group_ids != parent_ids)
    following = torch.nn.functional.pad(group_ids[:, 1:], (0, 1), value=-1)
    terminal = branch & (group_ids != following)
    scored = real & torch.isfinite(logprobs)
    seq = group_ids.shape[1]
    pos = torch.arange(seq).expand_as(group_ids)
    gid = torch.where(real, group_ids, 0).long()
    span = int(gid.max()) + 1 if gid.numel() else 1
    last_scored = torch.full((group_ids.shape[0], span), -1, dtype=torch.long)
    last_scored.scatter_reduce_(1, gid, torch.where(scored, pos, -1), reduce="amax")
    no_later_score = last_scored.gather(1, gid) <= pos
    return terminal | (branch & no_later_score)


def build_moe_routing_replay_bundle_from_packed_tensors(
        *, packed_tensors: Mapping[str, Any], global_grad_accumulation_sequences: int,
        topology: ParallelTopology | None = None) -> MoeRoutingReplayBundle:
    """A bundle with one step per ``global_grad_accumulation_sequences``
    packed sequences, one router per MoE layer and one call per sequence
    (the micro of its sample); step slots past the last sequence become
    padded micro slots of synthetic routes.

    ``packed_tensors["moe_routing_replay"]`` has ``expert_indices`` [S, seq,
    L, k], ``token_mask`` [S, seq] (route captured) and ``num_experts``;
    ``group_ids`` / ``parent_ids`` / ``logprobs`` [S, seq] decide which
    uncaptured rows are acceptable (padding and the rows of
    ``_route_free_rows``) and get synthetic routes.
    """
    rr = packed_tensors.get("moe_routing_replay")
    if rr is None:
        raise RuntimeError("Packed tensors do not contain MoE routing replay data")
    per_step = int(global_grad_accumulation_sequences)
    if per_step <= 0:
        raise RuntimeError(f"global_grad_accumulation_sequences must be positive, got {per_step}")
    ids = rr.expert_indices
    captured = rr.token_mask.bool()
    n_seq, seq, n_layers, k = (int(d) for d in ids.shape)
    e = int(rr.num_experts)
    gids = packed_tensors["group_ids"]
    bad = (gids != -1) & ~captured & ~_route_free_rows(gids, packed_tensors["parent_ids"],
                                                       packed_tensors["logprobs"])
    if bool(bad.any()):
        raise RuntimeError("Packed tensors are missing MoE routes outside terminal completion "
                           f"tokens ({int(bad.sum())} rows)")
    keys = [f"chunk_00.layer_{layer:04d}.mlp.router" for layer in range(n_layers)]
    n_steps = math.ceil(n_seq / per_step)
    steps: dict[int, StepRoutes] = {}
    for step in range(n_steps):
        routers: dict[str, StepRouterRoutes] = {}
        for layer, rk in enumerate(keys):
            calls: dict[int, RouterCallRoute] = {}
            for slot in range(per_step):
                sample = step * per_step + slot
                if sample < n_seq:
                    rows = ids[sample, :, layer, :].to(torch.int32).clone()
                    holes = torch.nonzero(~captured[sample]).flatten()
                    if holes.numel():
                        rows[holes] = synthetic_replay_rows(
                            row_positions=holes, num_experts=e, topk=k, dtype=torch.int32,
                            seed=(sample + 1) * _SEED_SAMPLE + (layer + 1) * _SEED_LAYER)
                    meta = {"sample_index": sample}
                else:
                    rows = synthetic_replay_rows(
                        row_positions=range(seq), num_experts=e, topk=k, dtype=torch.int32,
                        seed=(step + 1) * _SEED_SAMPLE + (layer + 1) * _SEED_LAYER
                        + (slot + 1) * _SEED_SLOT)
                    meta = {"micro_slot": slot}
                calls[slot] = RouterCallRoute(expert_indices=rows,
                                              expert_mask=torch.ones_like(rows, dtype=torch.bool),
                                              num_experts=e, **meta)
            routers[rk] = StepRouterRoutes(calls=calls)
        steps[step] = StepRoutes(routers=routers,
                                 global_token_uids=torch.arange(seq, dtype=torch.int64))
    return MoeRoutingReplayBundle(topology=topology or parallel_topology_from_env(),
                                  num_steps=n_steps, max_topk=k, router_keys=keys, steps=steps)


# ------------------------------------------------- device replay target type
class DeviceReplayTarget:
    """A replay target in device memory: token t replays ``table[rows[t]]``
    (rows[t] >= 0) or ``extra[-rows[t] - 1]`` (rows[t] < 0, synthetic rows);
    table / extra int32 [N, k] / [X, k], rows int32 [T].  The HIP replay
    kernel reads it as it is (``ops.router_replay_rows``)."""

    def __init__(self, table: torch.Tensor, rows: torch.Tensor,
                 extra: torch.Tensor | None = None) -> None:
        if table.dim() != 2 or rows.dim() != 1 or (extra is not None and extra.dim() != 2):
            raise RuntimeError("DeviceReplayTarget takes a table [N, k], rows [T] and an "
                               "optional extra table [X, k]")
        self.table, self.rows, self.extra = table, rows, extra

    @property
    def shape(self) -> torch.Size:
        return torch.Size((int(self.rows.shape[0]), int(self.table.shape[1])))

    @property
    def device(self) -> torch.device:
        return self.table.device

    def materialize(self) -> torch.Tensor:
        """The [T, k] int64 target ids."""
        r = self.rows.long()
        out = self.table.index_select(0, r.clamp_min(0)).long()
        if self.extra is not None and bool((r < 0).any()):
            side = self.extra.index_select(0, (-r - 1).clamp(0, self.extra.shape[0] - 1)).long()
            out = torch.where((r < 0).unsqueeze(1), side, out)
        return out


# -------------------------------------------------- megatron RouterReplay API
class RouterReplayAction(enum.Enum):
    RECORD = "record"
    REPLAY_FORWARD = "replay_forward"
    REPLAY_BACKWARD = "replay_backward"


class RouterReplay:
    """Replay state of one router with megatron's ``RouterReplay`` interface:
    under REPLAY_FORWARD the target set with ``set_target_indices`` replaces
    the top-k selection.  The class-level calls act on every live instance."""

    _live: "weakref.WeakSet[RouterReplay]" = weakref.WeakSet()

    def __init__(self) -> None:
        self.target_topk_idx: torch.Tensor | DeviceReplayTarget | None = None
        self.recorded_topk_idx: torch.Tensor | None = None
        self.router_replay_action: RouterReplayAction | None = None
        RouterReplay._live.add(self)

    @staticmethod
    def clear_global_indices() -> None:
        for r in list(RouterReplay._live):
            r.clear_indices()

    @staticmethod
    def set_global_router_replay_action(action: RouterReplayAction) -> None:
        for r in list(RouterReplay._live):
            r.router_replay_action = action

    @staticmethod
    def clear_global_router_replay_action() -> None:
        RouterReplay.set_global_router_replay_action(None)

    def set_target_indices(self, topk_indices) -> None:
        self.target_topk_idx = topk_indices

    def set_router_replay_action(self, action: RouterReplayAction | None) -> None:
        self.router_replay_action = action

    def clear_router_replay_action(self) -> None:
        self.router_replay_action = None

    def clear_indices(self) -> None:
        self.target_topk_idx = self.recorded_topk_idx = None

    def record_indices(self, topk_indices: torch.Tensor) -> None:
        self.recorded_topk_idx = topk_indices.detach()

    def get_recorded_indices(self) -> torch.Tensor | None:
        return self.recorded_topk_idx

    def active_target(self):
        """The target replacing top-k now (None unless REPLAY_FORWARD)."""
        return self.target_topk_idx if self.router_replay_action is RouterReplayAction.REPLAY_FORWARD \
            else None

    def get_replay_topk(self, scores: torch.Tensor, topk: int, num_groups: int | None = None,
                        group_topk: int | None = None,
                        default_compute_topk: Callable[..., Any] | None = None):
        """(selected scores, ids): the target's under REPLAY_FORWARD, otherwise
        ``default_compute_topk`` (recorded under RECORD)."""
        target = self.active_target()
        if target is not None:
            if isinstance(target, DeviceReplayTarget):
                target = target.materialize()
            ids = target.to(device=scores.device, dtype=torch.long)
            return scores.gather(1, ids), ids
        vals, ids = default_compute_topk(scores, topk, num_groups, group_topk)
        if self.router_replay_action is RouterReplayAction.RECORD:
            self.record_indices(ids)
        return vals, ids


# ---------------------------------------------------------- parallel layout
class SingleProcessParallelState:
    """The parallel_state queries the replay needs, for one process on one GPU."""

    def get_tensor_model_parallel_world_size(self) -> int:
        return 1

    def get_tensor_model_parallel_rank(self) -> int:
        return 0

    def get_context_parallel_world_size(self) -> int:
        return 1

    def get_context_parallel_rank(self) -> int:
        return 0

    def get_data_parallel_world_size(self) -> int:
        return 1

    def get_data_parallel_rank(self) -> int:
        return 0


class TopologyAwareLocalTokenIndexer:
    """This rank's token uids of a packed sequence: the context-parallel
    share (chunks r and 2cp-1-r of 2cp equal chunks, megatron's load-balanced
    split) and, with sequence parallelism, the tensor-parallel rank's slice."""

    def __init__(self, parallel_state_module: Any | None = None) -> None:
        self._ps = parallel_state_module or SingleProcessParallelState()

    def build_local_token_uids(self, *, global_token_uids: torch.Tensor, num_local_tokens: int,
                               sequence_parallel: bool, context_parallel_size: int) -> torch.Tensor:
        uids = global_token_uids.detach().to(device="cpu", dtype=torch.int64).reshape(-1)
        cp = int(self._ps.get_context_parallel_world_size())
        if context_parallel_size > 1 and cp > 1:
            chunks = uids.chunk(2 * cp)
            r = int(self._ps.get_context_parallel_rank())
            uids = torch.cat((chunks[r], chunks[2 * cp - 1 - r]))
        tp = int(self._ps.get_tensor_model_parallel_world_size())
        if sequence_parallel and tp > 1 and uids.numel() != num_local_tokens:
            if uids.numel() % tp or uids.numel() // tp != num_local_tokens:
                raise RuntimeError(f"{uids.numel()} token uids cannot be split over {tp} "
                                   f"sequence-parallel ranks into {num_local_tokens} each")
            r = int(self._ps.get_tensor_model_parallel_rank())
            uids = uids[r * num_local_tokens:(r + 1) * num_local_tokens]
        if uids.numel() != num_local_tokens:
            raise RuntimeError(f"expected {num_local_tokens} local token uids, got {uids.numel()}")
        return uids.contiguous()


# ------------------------------------------------------------- controller parts
MicroKey = tuple[str, int]


class _CallCursor:
    """Consumption of one router's calls in a step.

    ``plan`` lists the call indices this rank runs, in order, and ``keys``
    the micro each belongs to.  ``pending(active)`` is what the active micro
    may run next; ``take(active)`` consumes it.  A call for the micro that
    just consumed its route, when the plan has moved on to another micro, is
    an activation recompute: it gets that route again."""

    def __init__(self, plan: list[int], keys: list[MicroKey | None]) -> None:
        self.plan, self.keys = plan, keys
        self.pos = 0
        self.last: tuple[int, MicroKey | None] | None = None
        self.reuses = 0

    def _recompute(self, active: MicroKey | None) -> bool:
        return (active is not None and self.last is not None and self.last[1] == active
                and (self.pos == len(self.plan) or self.keys[self.pos] != active))

    def pending(self, active: MicroKey | None) -> list[int]:
        if self._recompute(active):
            return [self.last[0]]
        if self.pos == len(self.plan):
            return []
        if active is None:
            return [self.plan[self.pos]]
        run = []
        for ci, key in zip(self.plan[self.pos:], self.keys[self.pos:]):
            if key != active:
                break
            run.append(ci)
        return run

    def take(self, active: MicroKey | None, allow_reuse: bool, where: str) -> int:
        if self._recompute(active):
            if not allow_reuse:
                raise RuntimeError(f"{where}: recompute reuse is disabled, yet micro {active} "
                                   "ran its router again")
            self.reuses += 1
            return self.last[0]
        if self.pos == len(self.plan):
            raise RuntimeError(f"{where}: more router calls than the {len(self.plan)} planned")
        ci = self.plan[self.pos]
        self.last = (ci, self.keys[self.pos])
        self.pos += 1
        return ci

    @property
    def done(self) -> bool:
        return self.pos == len(self.plan)


class _UidRows:
    """Row of each token uid in the step's route tables.  Dense uid ranges
    (the packed-sequence case) map by an offset; others through a sorted
    index (searchsorted), vectorised either way.  Negative uids (tokens
    without one) map to -1 - (their rank among the negative positions), the
    side-table convention of the replay kernel."""

    def __init__(self, uids: torch.Tensor) -> None:
        self.n = int(uids.numel())
        self.dense = None
        if self.n and bool((uids[1:] - uids[:-1] == 1).all()):
            self.dense = int(uids[0])
        else:
            self.sorted, self.order = torch.sort(uids)

    def rows(self, uids: torch.Tensor, where: str) -> tuple[torch.Tensor, torch.Tensor]:
        """(rows int64 [T], positions of the negative uids)."""
        neg = torch.nonzero(uids < 0).flatten()
        rows = torch.empty_like(uids)
        valid = uids >= 0
        v = uids[valid]
        if self.dense is not None:
            r = v - self.dense
            bad = (r < 0) | (r >= self.n)
            if bool(bad.any()):
                raise RuntimeError(f"{where}: token uid {int(v[bad][0])} is outside the active "
                                   f"dense step span [{self.dense}, {self.dense + self.n})")
        else:
            at = torch.searchsorted(self.sorted, v).clamp_max(max(self.n - 1, 0))
            bad = (self.sorted[at] != v) if self.n else torch.ones_like(v, dtype=torch.bool)
            if bool(bad.any()):
                raise RuntimeError(f"{where}: token uid {int(v[bad][0])} is missing from the "
                                   "step's global_token_uids")
            r = self.order[at]
        rows[valid] = r
        rows[neg] = -1 - torch.arange(neg.numel())
        return rows, neg


@dataclass
class _Binding:
    key: str
    module: Any
    original_routing: Any
    replay: Any
    topk: int
    sequence_parallel: bool


@dataclass
class _Micro:
    """Targets staged for one micro: per uid layout, per router."""
    uid_sets: dict[str, torch.Tensor] = field(default_factory=dict)
    targets: dict[tuple[str, str], Any] = field(default_factory=dict)  # (layout, router) -> target
    calls: dict[str, int] = field(default_factory=dict)               # router -> call staged
    active: str | None = None
    ready: Any = None          # event after the side-stream copies (device targets)
    installed: dict[str, tuple[str, int]] = field(default_factory=dict)


class MoeRoutingReplayController:
    """Drives megatron-style routers to replay a bundle's routes.

    Per step: ``set_step`` (validate, plan each router's calls, upload the
    step's route table) -> per micro ``begin_micro`` + ``set_local_input_token_uids``
    / ``prepare_micro_targets`` (uids -> rows, targets staged) -> each router's
    ``routing`` installs its target -> ``finalize_step`` checks that every
    planned call ran.  ``device_targets`` (CUDA) hands the routers
    ``DeviceReplayTarget`` views for the HIP replay kernel; otherwise targets
    are [T, k] int64 tensors on ``device``.
    """

    def __init__(self, *, bundle: MoeRoutingReplayBundle, strict: bool,
                 local_token_indexer: Any | None = None, allow_recompute_reuse: bool = True,
                 device: torch.device | str | None = None, parallel_state: Any | None = None,
                 device_targets: bool = False) -> None:
        self.bundle = bundle
        self.strict = strict
        self.allow_recompute_reuse = allow_recompute_reuse
        self.device_targets = device_targets
        self.parallel_state = parallel_state or SingleProcessParallelState()
        self.local_token_indexer = local_token_indexer or TopologyAwareLocalTokenIndexer(
            self.parallel_state)
        self._device = torch.device(device) if device is not None else None
        self._bindings: dict[str, _Binding] = {}
        self._copy_stream: torch.cuda.Stream | None = None
        self._clear_step()

    # ------------------------------------------------------------ state
    def _clear_step(self) -> None:
        self._step: int | None = None
        self._routes: StepRoutes | None = None
        self._cursors: dict[str, _CallCursor] = {}
        self._uid_rows: _UidRows | None = None
        self._tables: dict[tuple[str, int], torch.Tensor] = {}   # device views per call
        self._micro_key: MicroKey | None = None
        self._micro_order: int | None = None
        self._micro = _Micro()

    def _device_for_targets(self) -> torch.device:
        if self._device is not None:
            return self._device
        return torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() \
            else torch.device("cpu")

    def _on_gpu(self) -> bool:
        return self.device_targets and self._device_for_targets().type == "cuda"

    def call_plan(self, router_key: str) -> list[int]:
        """Call indices router ``router_key`` consumes this step, in order."""
        return list(self._cursors[router_key].plan)

    def update_bundle(self, *, bundle: MoeRoutingReplayBundle, strict: bool) -> None:
        self.bundle, self.strict = bundle, strict
        self.clear_replay_state()
        if strict:
            absent = sorted(k for k in self._bindings if k not in bundle.router_keys)
            if absent:
                raise RuntimeError(f"Router keys from model are missing in replay bundle: {absent}")

    def clear_replay_state(self) -> None:
        RouterReplay.clear_global_indices()
        RouterReplay.clear_global_router_replay_action()
        self._clear_step()

    # ------------------------------------------------------------ patching
    def install_router_patches(self, model_chunks: list[Any]) -> None:
        """Wrap ``routing`` of every ``*.mlp.router`` module so that its replay
        target is installed right before it runs."""
        global _installed
        if self._bindings:
            return
        for chunk_index, chunk in enumerate(model_chunks):
            for name, module in chunk.named_modules():
                if ROUTER_NAME_TOKEN not in name or not hasattr(module, "routing"):
                    continue
                key = build_router_key_from_module_name(chunk_index=chunk_index, module_name=name)
                cfg = getattr(module, "config", None)
                replay = getattr(module, "router_replay", None)
                problem = None
                if self.strict and key not in self.bundle.router_keys:
                    problem = "its key is not in the replay bundle"
                elif getattr(cfg, "moe_router_fusion", False):
                    problem = ("replay needs moe_router_fusion=False (the fused router bypasses "
                               "RouterReplay)")
                elif replay is None:
                    problem = ("replay needs the model built with "
                               "provider.moe_enable_routing_replay=True (no router_replay)")
                elif getattr(module, "_art_routing_replay_target_patched", False):
                    problem = "its routing is already patched"
                if problem:
                    raise RuntimeError(f"router '{key}': {problem}")
                original = module.routing
                hook = torch.compiler.disable(lambda _k=key: self._install_target(_k))

                def routing(mod, *args, _orig=original, _hook=hook, **kwargs):
                    _hook()
                    return _orig(*args, **kwargs)

                module.routing = types.MethodType(routing, module)
                module._art_routing_replay_target_patched = True
                self._bindings[key] = _Binding(key, module, original, replay, int(module.topk),
                                               bool(getattr(cfg, "sequence_parallel", False)))
        _installed = weakref.ref(self)

    def remove_router_patches(self) -> None:
        global _installed
        if active_routing_replay_controller() is self:
            _installed = None
        for b in self._bindings.values():
            b.module.routing = b.original_routing
            if hasattr(b.module, "_art_routing_replay_target_patched"):
                del b.module._art_routing_replay_target_patched
        self._bindings.clear()
        self.clear_replay_state()

    # ------------------------------------------------------------ steps
    def _micro_key_of(self, sample: int | None, local_micro: int) -> MicroKey:
        if sample is not None:
            return ("sample", int(sample))
        ps = self.parallel_state
        return ("dummy_micro_slot",
                local_micro * int(ps.get_data_parallel_world_size()) + int(ps.get_data_parallel_rank()))

    def _plan(self, rk: str, sample_index, per_step: int | None) -> list[int]:
        calls = self._routes.routers[rk].calls
        where = f"step {self._step} router '{rk}'"
        if all(r.call_key is not None for r in calls.values()):
            by_micro: dict[MicroKey, list[int]] = {}
            for ci in sorted(calls):
                by_micro.setdefault(calls[ci].call_key, []).append(ci)
            samples = sample_index if isinstance(sample_index, list) else [sample_index]
            plan: list[int] = []
            for local, sample in enumerate(samples):
                key = self._micro_key_of(sample, local)
                if key not in by_micro:
                    raise RuntimeError(f"{where}: no calls for micro {key}")
                plan += by_micro[key]
            return plan
        # legacy layout (no per-call micro metadata): contiguous blocks per sample
        n = len(calls)
        if sample_index is None:
            if n != 1:
                raise RuntimeError(f"{where}: the bundle lacks sample metadata and has {n} calls")
            return [0]
        samples = [s for s in (sample_index if isinstance(sample_index, list) else [sample_index])
                   if s is not None]
        count = per_step if per_step is not None else (
            len(samples) if isinstance(sample_index, list) else 1)
        if count <= 0 or n % count:
            raise RuntimeError(f"{where}: {n} router calls are not divisible by the step's "
                               f"{count} samples")
        each = n // count
        plan = []
        for s in samples:
            off = int(s) - self._step * count
            if not 0 <= off < count:
                raise RuntimeError(f"{where}: sample {s} is outside the step's samples "
                                   f"[{self._step * count}, {self._step * count + count})")
            plan += range(off * each, off * each + each)
        return plan

    def set_step(self, *, step_index: int, sample_index: int | list[int | None] | None,
                 global_grad_accumulation_sequences: int | None = None) -> None:
        """Start step ``step_index`` for this rank's samples (one per local micro;
        None for a padded micro slot)."""
        if step_index not in self.bundle.steps:
            raise RuntimeError(f"Replay bundle missing step_index={step_index}; it has steps "
                               f"{sorted(self.bundle.steps)}")
        self._clear_step()
        self._step, self._routes = step_index, self.bundle.steps[step_index]
        for rk in sorted(self._bindings):
            if rk not in self._routes.routers:
                raise RuntimeError(f"step {step_index} has no routes for router '{rk}'")
            topk = self._bindings[rk].topk
            for ci, route in self._routes.routers[rk].calls.items():
                if not bool(route.expert_mask.all()):
                    raise RuntimeError(f"masked slots are unsupported by native MoE routing replay "
                                       f"(step {step_index}, router '{rk}', call {ci})")
                if route.max_topk != topk:
                    raise RuntimeError(f"replayed route topk does not match the router: step "
                                       f"{step_index}, router '{rk}', call {ci} has "
                                       f"{route.max_topk}, the router {topk}")
            plan = self._plan(rk, sample_index, global_grad_accumulation_sequences)
            calls = self._routes.routers[rk].calls
            self._cursors[rk] = _CallCursor(plan, [calls[ci].call_key for ci in plan])
        self._uid_rows = _UidRows(self._routes.global_token_uids)
        if self._on_gpu() and self._bindings:
            self._upload_step_table()
        RouterReplay.clear_global_indices()
        RouterReplay.set_global_router_replay_action(RouterReplayAction.REPLAY_FORWARD)

    def finalize_step(self) -> None:
        """Check that every router consumed exactly its planned calls."""
        if self._routes is None:
            raise RuntimeError("finalize_step called before set_step")
        for rk, cur in sorted(self._cursors.items()):
            if not cur.done:
                raise RuntimeError(f"Routing replay step consumption mismatch: step {self._step}, "
                                   f"router '{rk}' ran {cur.pos} of {len(cur.plan)} planned calls")
        reused = {rk: c.reuses for rk, c in self._cursors.items() if c.reuses}
        if reused:
            logger.info("routing replay step %s: routes reused for recompute %s", self._step, reused)
        self.clear_replay_state()

    # ------------------------------------------------------------ micros
    def begin_micro(self, sample_index: int | None, micro_order: int) -> None:
        """Make micro ``micro_order`` (of ``sample_index``) the active one; each
        router must have exactly one call for it."""
        self._micro_key = self._micro_key_of(sample_index, micro_order)
        self._micro_order = micro_order
        for rk in sorted(self._cursors):
            pending = self._cursors[rk].pending(self._micro_key)
            if len(pending) != 1:
                raise RuntimeError(f"Routing replay expected exactly one router call per micro for "
                                   f"router '{rk}', got calls {pending}")

    def set_local_input_token_uids(self, local_token_uids: torch.Tensor | None) -> None:
        self.prepare_micro_targets({"attention": local_token_uids})

    def prepare_micro_targets(self, token_uid_sets: Mapping[str, torch.Tensor | None], *,
                              active_token_uid_key: str = "attention") -> None:
        """Stage the active micro's targets for each token layout (e.g. the
        attention order and a linear-attention order of the same tokens)."""
        if self._routes is None or self._micro_order is None:
            raise RuntimeError("target staging needs set_step and begin_micro first")
        sets = {}
        for name, uids in token_uid_sets.items():
            if uids is None:
                continue
            if uids.device.type != "cpu":
                raise RuntimeError("token uids must be CPU metadata (a device tensor would force "
                                   "a host sync in the model path)")
            sets[name] = uids.detach().to(torch.int64).reshape(-1).contiguous()
        if active_token_uid_key not in sets:
            raise RuntimeError(f"token uid layout '{active_token_uid_key}' was not given "
                               f"(got {sorted(sets)})")
        self._micro = _Micro(uid_sets=sets)
        for rk in sorted(self._bindings):
            pending = self._cursors[rk].pending(self._micro_key)
            if len(pending) != 1:
                raise RuntimeError(f"Routing replay expected exactly one router call per micro for "
                                   f"router '{rk}', got calls {pending}")
            self._micro.calls[rk] = pending[0]
        if self._on_gpu():
            self._stage_on_device()
        else:
            self._stage_on_host()
        self.set_active_token_uid_key(active_token_uid_key)

    def set_active_token_uid_key(self, token_uid_key: str) -> None:
        if self._bindings and token_uid_key not in self._micro.uid_sets:
            raise RuntimeError(f"token uid layout '{token_uid_key}' was not staged for this micro "
                               f"(staged: {sorted(self._micro.uid_sets)})")
        self._micro.active = token_uid_key

    def local_token_uids_for_active_dispatch(self, *, num_local_tokens: int,
                                             sequence_parallel: bool) -> torch.Tensor | None:
        """The active layout's uids as this rank dispatches them (padding
        dropped when that is what makes the count match), or None."""
        uids = self._micro.uid_sets.get(self._micro.active) if self._micro.active else None
        if uids is None:
            return None
        local = self._sp_slice(uids, sequence_parallel)
        if local.numel() == num_local_tokens:
            return local
        real = local[local >= 0]
        return real.contiguous() if real.numel() == num_local_tokens else None

    def _sp_slice(self, uids: torch.Tensor, sequence_parallel: bool) -> torch.Tensor:
        """A sequence-parallel router sees its tensor-parallel rank's
        ceil(T / tp) tokens, the last rank's share padded with -1."""
        tp = int(self.parallel_state.get_tensor_model_parallel_world_size())
        if not sequence_parallel or tp <= 1:
            return uids
        share = -(-uids.numel() // tp)
        part = uids[int(self.parallel_state.get_tensor_model_parallel_rank()) * share:][:share]
        out = uids.new_full((share,), -1)
        out[:part.numel()] = part
        return out

    def _synthetic(self, call: int, positions: torch.Tensor, e: int, k: int) -> torch.Tensor:
        return synthetic_replay_rows(
            row_positions=positions, num_experts=e, topk=k, dtype=torch.int32,
            seed=(int(self._step or 0) + 1) * _SEED_SAMPLE + (call + 1) * _SEED_LAYER)

    def _stage_on_host(self) -> None:
        dev = self._device_for_targets()
        for name, uids in self._micro.uid_sets.items():
            for rk, b in self._bindings.items():
                ci = self._micro.calls[rk]
                route = self._routes.routers[rk].calls[ci]
                where = f"step {self._step} router '{rk}' call {ci}"
                local = self._sp_slice(uids, b.sequence_parallel)
                rows, neg = self._uid_rows.rows(local, where)
                if bool((rows >= route.num_global_tokens).any()):
                    raise RuntimeError(f"{where}: a token row is past the route's "
                                       f"{route.num_global_tokens} rows")
                src = route.expert_indices
                target = src.index_select(0, rows.clamp_min(0).to(src.device)).long()
                if neg.numel():
                    target[neg.to(src.device)] = self._synthetic(
                        ci, neg, route.num_experts, route.max_topk).long().to(src.device)
                if dev.type == "cuda" and target.device.type == "cpu":
                    target = self._upload(target)
                self._micro.targets[(name, rk)] = target
        if dev.type == "cuda" and self._micro.targets:
            ready = torch.cuda.Event()
            ready.record(self._side_stream())
            self._micro.ready = ready

    # ------------------------------------------------------------ device side
    def _side_stream(self) -> torch.cuda.Stream:
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=self._device_for_targets())
        return self._copy_stream

    def _upload(self, host: torch.Tensor) -> torch.Tensor:
        """Device copy of ``host`` made on the side stream (after the compute
        stream's queued work, which may still read the buffer's last owner)."""
        dev = self._device_for_targets()
        side = self._side_stream()
        buf = torch.empty(host.shape, dtype=host.dtype, device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            buf.copy_(host.pin_memory(), non_blocking=True)
        buf.record_stream(side)
        return buf

    def _upload_step_table(self) -> None:
        """Every call this rank will consume, all routers, in one device table
        per topk: one host-to-device copy per step."""
        by_k: dict[int, list[tuple[str, int, RouterCallRoute]]] = {}
        for rk, cur in sorted(self._cursors.items()):
            for ci in dict.fromkeys(cur.plan):
                route = self._routes.routers[rk].calls[ci]
                by_k.setdefault(route.max_topk, []).append((rk, ci, route))
        dev = self._device_for_targets()
        for k, entries in by_k.items():
            if all(r.expert_indices.device == dev for _, _, r in entries):
                for rk, ci, route in entries:     # loaded straight into device tables
                    self._tables[(rk, ci)] = route.expert_indices
                continue
            table = self._upload(torch.cat([r.expert_indices.cpu() for _, _, r in entries]))
            base = 0
            for rk, ci, route in entries:
                n = route.num_global_tokens
                self._tables[(rk, ci)] = table[base:base + n]
                base += n

    def _stage_on_device(self) -> None:
        """Row maps once per (layout, sequence-parallel slicing), shared by all
        routers; synthetic side tables per call when some tokens lack a uid."""
        maps: dict[tuple[str, bool], tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = {}
        for name, uids in self._micro.uid_sets.items():
            for rk, b in self._bindings.items():
                ci = self._micro.calls[rk]
                route = self._routes.routers[rk].calls[ci]
                where = f"step {self._step} router '{rk}' call {ci}"
                mk = (name, b.sequence_parallel)
                if mk not in maps:
                    rows, neg = self._uid_rows.rows(self._sp_slice(uids, b.sequence_parallel), where)
                    maps[mk] = (self._upload(rows.to(torch.int32)), neg,
                                rows.max() if rows.numel() else torch.tensor(-1))
                rows_dev, neg, top = maps[mk]
                if int(top) >= route.num_global_tokens:
                    raise RuntimeError(f"{where}: a token row is past the route's "
                                       f"{route.num_global_tokens} rows")
                extra = None
                if neg.numel():
                    extra = self._upload(self._synthetic(ci, neg, route.num_experts,
                                                         route.max_topk))
                self._micro.targets[(name, rk)] = DeviceReplayTarget(self._tables[(rk, ci)],
                                                                      rows_dev, extra)
        ready = torch.cuda.Event()
        ready.record(self._side_stream())
        self._micro.ready = ready

    def wait_for_staged_targets(self) -> None:
        """Order the compute stream after the staged targets' copies."""
        if self._micro.ready is not None:
            torch.cuda.current_stream(self._device_for_targets()).wait_event(self._micro.ready)
            self._micro.ready = None

    # ------------------------------------------------------------ at routing time
    def _install_target(self, router_key: str) -> None:
        """Runs right before router ``router_key`` routes: consume its call and
        give its RouterReplay the staged target."""
        m = self._micro
        if self._routes is None or self._micro_order is None or m.active is None:
            raise RuntimeError(f"router '{router_key}' ran before its replay targets were staged")
        cur = self._cursors[router_key]
        pending = cur.pending(self._micro_key)
        if len(pending) != 1:
            raise RuntimeError(f"Routing replay expected exactly one router call per micro for "
                               f"router '{router_key}', got calls {pending}")
        ci = cur.take(self._micro_key, self.allow_recompute_reuse,
                      f"step {self._step} router '{router_key}'")
        if ci != m.calls.get(router_key):
            raise RuntimeError(f"router '{router_key}' consumed call {ci}, staged "
                               f"{m.calls.get(router_key)}")
        if m.installed.get(router_key) == (m.active, ci):
            return                                   # recompute: target already in place
        self.wait_for_staged_targets()
        target = m.targets[(m.active, router_key)]
        b = self._bindings[router_key]
        if int(target.shape[1]) != b.topk:
            raise RuntimeError(f"router '{router_key}': staged target topk {int(target.shape[1])} "
                               f"!= router topk {b.topk}")
        b.replay.set_target_indices(target)
        b.replay.set_router_replay_action(RouterReplayAction.REPLAY_FORWARD)
        m.installed[router_key] = (m.active, ci)
