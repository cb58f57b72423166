"""vLLM route capture: the experts each token was routed to at sampling time,
aligned onto the trainer's tokenisation of the same conversation.

Mirrors ``art.preprocessing.moe_routing`` (/root/reference/src/art/preprocessing/
moe_routing.py): the metadata key ``art_moe_routing`` under which a choice
carries its routes, the response fields vLLM fills (``prompt_token_ids``,
``completion_token_ids`` / ``token_ids`` / ``output_token_ids``,
``prompt_routed_experts``, ``completion_routed_experts``, ``routed_experts``,
the latter also as a base64 ``.npy`` of rank 3), the public functions and the
error texts the reference's tests match are interface and stay as they are.

How it works here.  A token route is ``[layers][topk]`` expert ids.  Each
choice's prompt and completion routes are turned into one int64 array
``[tokens, layers, topk]`` up front (``np.asarray`` validates that they are
rectangular), token ids are compared as arrays, and the overlay onto the
tokenised sequence counts conflicting slots with one vectorised comparison
per choice instead of a Python loop per slot.  The aligned result is handed
back as nested lists, the type the packer and the reference's callers use.
"""
from __future__ import annotations

import base64
import io
from collections.abc import Mapping
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

ART_MOE_ROUTING_METADATA_KEY = "art_moe_routing"

PROMPT_TOKEN_IDS_KEY = "prompt_token_ids"
COMPLETION_TOKEN_IDS_KEY = "completion_token_ids"
PROMPT_ROUTED_EXPERTS_KEY = "prompt_routed_experts"
COMPLETION_ROUTED_EXPERTS_KEY = "completion_routed_experts"
ROUTED_EXPERTS_KEY = "routed_experts"

# fields of a vLLM response (top level or per choice) that carry routing
_RESPONSE_FIELDS = (PROMPT_TOKEN_IDS_KEY, COMPLETION_TOKEN_IDS_KEY, "output_token_ids",
                    "token_ids", PROMPT_ROUTED_EXPERTS_KEY, COMPLETION_ROUTED_EXPERTS_KEY,
                    ROUTED_EXPERTS_KEY)
_EXPERT_FIELDS = (PROMPT_ROUTED_EXPERTS_KEY, COMPLETION_ROUTED_EXPERTS_KEY, ROUTED_EXPERTS_KEY)
# where the completion's token ids may sit, in order of preference
_COMPLETION_ID_FIELDS = (COMPLETION_TOKEN_IDS_KEY, "output_token_ids", "token_ids")

TokenRoute = list[list[int]]


@dataclass
class MoeRoutingAlignmentStats:
    choices_with_routing: int = 0
    routed_tokens: int = 0
    overlap_conflict_rows: int = 0
    overlap_conflict_slots: int = 0
    overlap_compared_slots: int = 0


@dataclass
class MoeRoutingPackStats:
    packed_tokens: int = 0
    prefix_tree_rows: int = 0
    prefix_tree_conflict_rows: int = 0
    prefix_tree_conflict_slots: int = 0
    prefix_tree_compared_slots: int = 0

    def add_alignment(self, stats: MoeRoutingAlignmentStats) -> None:
        self.prefix_tree_conflict_rows += stats.overlap_conflict_rows
        self.prefix_tree_conflict_slots += stats.overlap_conflict_slots
        self.prefix_tree_compared_slots += stats.overlap_compared_slots


@dataclass
class PackedMoeRoutingReplay:
    """Packed routes: ``expert_indices`` [sequences, seq_len, layers, topk]
    (int32), ``token_mask`` [sequences, seq_len] (route captured)."""
    expert_indices: Any
    token_mask: Any
    num_layers: int
    topk: int
    num_experts: int
    pack_stats: MoeRoutingPackStats = field(default_factory=MoeRoutingPackStats)

    def __post_init__(self) -> None:
        shape = tuple(self.expert_indices.shape)
        if len(shape) != 4:
            raise RuntimeError("expert_indices must have shape "
                               f"[num_sequences, sequence_length, num_layers, topk], got {shape}")
        if tuple(self.token_mask.shape) != shape[:2]:
            raise RuntimeError("token_mask shape must match packed route tokens, got "
                               f"{tuple(self.token_mask.shape)} vs {shape[:2]}")
        if self.num_layers != shape[2]:
            raise RuntimeError(f"num_layers={self.num_layers} does not match "
                               f"expert_indices.shape[2]={shape[2]}")
        if self.topk != shape[3]:
            raise RuntimeError(f"topk={self.topk} does not match expert_indices.shape[3]={shape[3]}")
        if self.num_experts <= 0:
            raise RuntimeError(f"num_experts must be >0, got {self.num_experts}")
        if self.topk > self.num_experts:
            raise RuntimeError("MoE routing topk cannot exceed num_experts: "
                               f"topk={self.topk}, num_experts={self.num_experts}")


# ------------------------------------------------------------ choice metadata
def _extra_of(choice: Any) -> dict | None:
    if isinstance(choice, Mapping):
        return choice  # type: ignore[return-value]
    return getattr(choice, "model_extra", None)


def _routing_fields(src: Mapping[str, Any]) -> dict[str, Any]:
    return {k: src[k] for k in _RESPONSE_FIELDS if k in src}


def _has_experts(meta: Mapping[str, Any]) -> bool:
    return any(meta.get(k) is not None for k in _EXPERT_FIELDS)


def attach_moe_routing_metadata_to_choice(*, choice: Any, response_payload: Mapping[str, Any],
                                          choice_index: int = 0) -> None:
    """Copy the routing fields of a vLLM response (top level, then choice
    ``choice_index``'s own, which take precedence) into the choice's extras
    under ``art_moe_routing``; nothing happens without routed experts."""
    meta = _routing_fields(response_payload)
    raw = response_payload.get("choices")
    if isinstance(raw, list) and choice_index < len(raw) and isinstance(raw[choice_index], Mapping):
        meta.update(_routing_fields(raw[choice_index]))
    if not meta or not _has_experts(meta):
        return
    extra = _extra_of(choice)
    if extra is None:
        raise RuntimeError("OpenAI Choice.model_extra is unavailable for route capture")
    extra[ART_MOE_ROUTING_METADATA_KEY] = meta


def choice_moe_routing_metadata(choice: Any) -> dict[str, Any] | None:
    """The routing fields a choice carries (nested under ``art_moe_routing``
    or at the top level of its extras), or None without routed experts."""
    extra = _extra_of(choice) or {}
    nested = extra.get(ART_MOE_ROUTING_METADATA_KEY)
    if isinstance(nested, Mapping):
        return dict(nested) if _has_experts(nested) else None
    top = _routing_fields(extra)
    return top if _has_experts(top) else None


# --------------------------------------------------------------- normalising
def _token_ids(raw: Any) -> np.ndarray:
    if raw is None:
        raise RuntimeError("Missing routed token ids")
    if not isinstance(raw, list):
        raise RuntimeError(f"Expected routed token ids list, got {type(raw)}")
    return np.asarray([int(t) for t in raw], dtype=np.int64)


def _completion_ids(meta: Mapping[str, Any]) -> np.ndarray:
    for key in _COMPLETION_ID_FIELDS:
        if key in meta:
            return _token_ids(meta[key])
    raise RuntimeError("Missing routed completion token ids")


def _decode_vllm_routed_experts(raw: str, *, field_name: str) -> np.ndarray:
    """vLLM's compact form: a base64-encoded ``.npy`` of shape
    [tokens, layers, topk] (loaded without pickle)."""
    try:
        arr = np.load(io.BytesIO(base64.b64decode(raw)), allow_pickle=False)
    except Exception as exc:
        raise RuntimeError(f"Failed to decode {field_name} as base64 .npy") from exc
    if arr.ndim != 3:
        raise RuntimeError(f"Expected {field_name} array with rank 3, got shape {arr.shape}")
    return arr


def _routes(raw: Any, *, field_name: str) -> np.ndarray:
    """[tokens, layers, topk] int64 routes of a response field (list form or
    base64 .npy); every token has the same non-zero layer count and topk."""
    if isinstance(raw, str):
        raw = _decode_vllm_routed_experts(raw, field_name=field_name)
    if raw is None:
        raise RuntimeError(f"Missing {field_name}")
    if isinstance(raw, np.ndarray):
        arr = raw
    else:
        if not isinstance(raw, list):
            raise RuntimeError(f"Expected {field_name} list, got {type(raw)}")
        for tok in raw:
            if not isinstance(tok, list):
                raise RuntimeError(f"Expected token route list in {field_name}")
            if not tok:
                raise RuntimeError("MoE token route cannot have zero layers")
            for layer in tok:
                if not isinstance(layer, list):
                    raise RuntimeError(f"Expected layer route list in {field_name}")
        try:
            arr = np.asarray(raw, dtype=np.int64)
        except ValueError:
            # ragged: say which rule broke, as the per-route check would
            for tok in raw:
                _check_route_shape(tok)
            raise RuntimeError(f"MoE routes in {field_name} differ in shape")
        if len(raw) == 0:
            arr = arr.reshape(0, 1, 1)
    if arr.ndim != 3 and arr.size:
        raise RuntimeError(f"Expected {field_name} routes of rank 3, got shape {arr.shape}")
    if arr.size and arr.shape[1] == 0:
        raise RuntimeError("MoE token route cannot have zero layers")
    if arr.size and arr.shape[2] == 0:
        raise RuntimeError("MoE token route cannot have zero topk")
    return arr.astype(np.int64, copy=False)


def _check_route_shape(route: TokenRoute) -> None:
    if not route:
        raise RuntimeError("MoE token route cannot have zero layers")
    k = len(route[0])
    if k <= 0:
        raise RuntimeError("MoE token route cannot have zero topk")
    if any(len(layer) != k for layer in route):
        raise RuntimeError("MoE token route topk must be constant across layers")


def _choice_routes(meta: Mapping[str, Any], n_prompt: int,
                   n_completion: int) -> tuple[np.ndarray, np.ndarray]:
    """(prompt routes, completion routes) of a choice: separate fields, or
    one ``routed_experts`` over prompt + completion (vLLM runs no forward for
    the last sampled token, so the completion may be one route short)."""
    if PROMPT_ROUTED_EXPERTS_KEY in meta:
        prompt = _routes(meta.get(PROMPT_ROUTED_EXPERTS_KEY), field_name=PROMPT_ROUTED_EXPERTS_KEY)
        for key in (COMPLETION_ROUTED_EXPERTS_KEY, ROUTED_EXPERTS_KEY):
            if key in meta:
                return prompt, _routes(meta[key], field_name=key)
        raise RuntimeError("Missing routed completion experts")
    both = _routes(meta.get(ROUTED_EXPERTS_KEY), field_name=ROUTED_EXPERTS_KEY)
    allowed = {n_prompt + n_completion, n_prompt + max(n_completion - 1, 0)}
    if len(both) not in allowed:
        raise RuntimeError("routed_experts length does not match prompt/completion token ids: "
                           f"{len(both)} not in {sorted(allowed)}")
    return both[:n_prompt], both[n_prompt:]


# ----------------------------------------------------------------- alignment
def align_choice_routes_to_tokenized_result(
        *, token_ids: list[int], choices: list[Any], choice_offsets: list[int],
        choice_token_lengths: list[int]) -> tuple[list[TokenRoute | None] | None,
                                                  MoeRoutingAlignmentStats]:
    """Per-token routes of a tokenised conversation from its choices' vLLM
    routing: choice i's prompt routes cover tokens [0, offset_i), its
    completion routes [offset_i, offset_i + length_i).  The first route seen
    for a token is kept; later overlapping routes only add to the conflict
    statistics.  Returns (None, stats) when no choice carries routing; a mix
    of routed and unrouted choices is an error."""
    if not (len(choices) == len(choice_offsets) == len(choice_token_lengths)):
        raise RuntimeError("Choice routing alignment inputs differ in length: "
                           f"choices={len(choices)}, offsets={len(choice_offsets)}, "
                           f"lengths={len(choice_token_lengths)}")
    ids = np.asarray([int(t) for t in token_ids], dtype=np.int64)
    n = ids.shape[0]
    table: np.ndarray | None = None        # [n, layers, topk] routes as aligned so far
    have = np.zeros(n, dtype=bool)
    stats = MoeRoutingAlignmentStats()
    routed = missing = False
    for choice, offset, length in zip(choices, choice_offsets, choice_token_lengths):
        meta = choice_moe_routing_metadata(choice)
        if meta is None:
            missing = True
            continue
        routed = True
        stats.choices_with_routing += 1
        p_ids, c_ids = _token_ids(meta.get(PROMPT_TOKEN_IDS_KEY)), _completion_ids(meta)
        p_routes, c_routes = _choice_routes(meta, len(p_ids), len(c_ids))
        want_p, want_c = ids[:offset], ids[offset:offset + length]
        if not np.array_equal(p_ids, want_p):
            raise RuntimeError("vLLM routed prompt token ids do not match ART-tokenized prefix: "
                               f"offset={offset}, vllm_len={len(p_ids)}, art_len={len(want_p)}")
        if not np.array_equal(c_ids, want_c):
            raise RuntimeError("vLLM routed completion token ids do not match ART-tokenized "
                               f"choice: offset={offset}, vllm_len={len(c_ids)}, "
                               f"art_len={len(want_c)}")
        if len(p_routes) != len(p_ids):
            raise RuntimeError("prompt_routed_experts length does not match prompt_token_ids: "
                               f"{len(p_routes)} != {len(p_ids)}")
        if len(c_routes) not in (len(c_ids), max(len(c_ids) - 1, 0)):
            raise RuntimeError("completion_routed_experts length does not match "
                               f"completion_token_ids: {len(c_routes)} != {len(c_ids)}")
        parts = [(0, r) for r in (p_routes,) if len(r)] + \
                [(offset, r) for r in (c_routes,) if len(r)]
        for start, routes in parts:
            if table is None:
                table = np.zeros((n,) + routes.shape[1:], dtype=np.int64)
            elif routes.shape[1:] != table.shape[1:]:
                raise RuntimeError("Cannot compare MoE routes with different shapes")
            pos = np.arange(start, start + len(routes))
            old = have[pos]
            if old.any():                  # overlap: count conflicting slots
                diff = table[pos[old]] != routes[old]
                slots = diff.reshape(diff.shape[0], -1)
                stats.overlap_compared_slots += int(slots.size)
                stats.overlap_conflict_slots += int(slots.sum())
                stats.overlap_conflict_rows += int(slots.any(axis=1).sum())
            new = ~old
            table[pos[new]] = routes[new]
            have[pos[new]] = True
        stats.routed_tokens = int(have.sum())
    if routed and missing:
        raise RuntimeError("Some trainable choices had MoE routes while others did not")
    if not routed:
        return None, stats
    aligned: list[TokenRoute | None] = [None] * n
    if table is not None:
        for i in np.nonzero(have)[0].tolist():
            aligned[i] = table[i].tolist()
    return aligned, stats


def count_route_slot_conflicts(left: TokenRoute, right: TokenRoute) -> tuple[int, int]:
    """(compared slots, differing slots) of two routes of one shape."""
    _check_route_shape(left)
    _check_route_shape(right)
    a, b = np.asarray(left, dtype=np.int64), np.asarray(right, dtype=np.int64)
    if a.shape != b.shape:
        raise RuntimeError("Cannot compare MoE routes with different shapes")
    return int(a.size), int((a != b).sum())


# ------------------------------------------------------------- tensorisation
def tensorize_moe_routes(routes_by_sequence: list[list[TokenRoute | None]],
                         seq_len: int) -> tuple[torch.Tensor, torch.Tensor, int, int, int]:
    """(expert_indices int32 [S, seq_len, layers, topk], token_mask bool
    [S, seq_len], layers, topk, num_experts) of packed per-token routes;
    tokens without a route (and padding) hold zeros with a false mask.
    ``num_experts`` is inferred as max(topk, largest id + 1).
    Follows pack.py:443-494 of the reference."""
    first = next((r for seq in routes_by_sequence for r in seq if r is not None), None)
    if first is None:
        raise RuntimeError("No MoE routes were packed")
    n_layers, k = len(first), len(first[0])
    out = np.zeros((len(routes_by_sequence), seq_len, n_layers, k), dtype=np.int32)
    mask = np.zeros((len(routes_by_sequence), seq_len), dtype=bool)
    top = 0
    for s, seq in enumerate(routes_by_sequence):
        pos = [i for i, r in enumerate(seq[:seq_len]) if r is not None]
        if not pos:
            continue
        try:
            block = np.asarray([seq[i] for i in pos], dtype=np.int64)
        except ValueError:
            block = None
        if block is None or block.shape[1:] != (n_layers, k):
            raise RuntimeError("Packed MoE routes must have one rectangular shape")
        out[s, pos] = block
        mask[s, pos] = True
        top = max(top, int(block.max()))
    return (torch.from_numpy(out), torch.from_numpy(mask), n_layers, k, max(k, top + 1))
