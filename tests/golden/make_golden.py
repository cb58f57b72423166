"""Write tests/golden/routing_kats.json.

The fixtures are known answers for the routing path, derived by hand from the
reference's own unit-test inputs (not produced by this build's oracle):

* replay routes of /root/reference/tests/unit/test_moe_routing_replay.py:40-55
  and :58-78 (E = 3, k = 2), with the expected routing map, tokens per expert,
  offsets, row -> token map and destination rows of the expert-major /
  token-ascending dispatch (megatron permute order);
* top-k tie / NaN / signed-zero rows under the build's documented tie rule
  (descending value, NaN highest, -0.0 == +0.0, lower expert id first);
* renormalised-softmax closed forms;
* the zero-token-expert counts and ranks of
  /root/reference/tests/integration/test_lora_quack_cutover.py:69-125;
* synthetic replay rows of ``_synthetic_replay_rows``
  (/root/reference/src/art/megatron/routing_replay.py:594-610) for seeds built
  with the formula at :538-539, produced by the Python standard library's
  ``random.Random(seed).sample`` (the reference calls the same stdlib routine).

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import random
from pathlib import Path

OUT = Path(__file__).with_name("routing_kats.json")


def synthetic_rows(positions, num_experts, topk, seed):
    # routing_replay.py:594-610
    return [random.Random(seed + (p + 1) * 1_299_709).sample(range(num_experts), topk)
            for p in positions]


def main() -> None:
    kats = {
        "replay_bundle_E3_k2": {
            "source": "tests/unit/test_moe_routing_replay.py:40-55",
            "num_experts": 3,
            "routes": [[0, 2], [1, 0], [2, 1], [1, 0]],
            "routing_map": [[1, 0, 1], [1, 1, 0], [0, 1, 1], [1, 1, 0]],
            "counts": [3, 3, 2],
            "offsets": [0, 3, 6, 8],
            "row_token": [0, 1, 3, 1, 2, 3, 0, 2],
            "dest": [[0, 6], [3, 1], [7, 4], [5, 2]],
        },
        "sampled_bundle_call0": {
            "source": "tests/unit/test_moe_routing_replay.py:58-78 (call 0)",
            "num_experts": 3,
            "routes": [[0, 2], [1, 0]],
            "counts": [2, 1, 1],
            "offsets": [0, 2, 3, 4],
            "row_token": [0, 1, 1, 0],
            "dest": [[0, 3], [2, 1]],
        },
        "sampled_bundle_call1": {
            "source": "tests/unit/test_moe_routing_replay.py:58-78 (call 1)",
            "num_experts": 3,
            "routes": [[2, 1], [0, 1]],
            "counts": [1, 2, 1],
            "offsets": [0, 1, 3, 4],
            "row_token": [1, 0, 1, 0],
            "dest": [[3, 1], [0, 2]],
        },
        "topk_tie_rule": [
            {"logits": [1.0, 3.0, 3.0, 2.0], "k": 2, "idx": [1, 2]},
            {"logits": [5.0, 5.0, 5.0, 5.0], "k": 3, "idx": [0, 1, 2]},
            {"logits": ["nan", 1.0, 2.0, 5.0], "k": 2, "idx": [0, 3]},
            {"logits": [0.0, "-0.0", 0.0, -1.0], "k": 2, "idx": [0, 1]},
            {"logits": ["-inf", -1.0, "inf", 3.0], "k": 3, "idx": [2, 3, 1]},
            {"logits": [2.0, 7.0, 7.0, "nan", "nan"], "k": 3, "idx": [3, 4, 1]},
        ],
        "softmax_closed_form": [
            {"logits": [0.0, math.log(3.0), -50.0], "k": 2, "idx": [1, 0], "w": [0.75, 0.25]},
            {"logits": [1.0, 1.0, 1.0, 1.0], "k": 4, "idx": [0, 1, 2, 3], "w": [0.25] * 4},
        ],
        "lora_cutover": {
            "source": "tests/integration/test_lora_quack_cutover.py:69-125",
            "counts": [32, 0, 16, 24],
            "in_features": 64,
            "out_features": 64,
            "ranks": [1, 3, 7, 16, 24],
            "seed_base": 20260323,
            "tolerance": {"atol": 5e-2, "rtol": 5e-2},
        },
        "synthetic_replay_rows": [],
    }
    for sample_index, layer_index, num_experts, topk in ((0, 0, 128, 8), (3, 5, 64, 4), (1, 47, 8, 2)):
        seed = (sample_index + 1) * 1_000_003 + (layer_index + 1) * 97_003
        positions = [0, 1, 7, 100]
        kats["synthetic_replay_rows"].append({
            "sample_index": sample_index, "layer_index": layer_index,
            "num_experts": num_experts, "topk": topk, "seed": seed,
            "positions": positions,
            "rows": synthetic_rows(positions, num_experts, topk, seed),
        })
    OUT.write_text(json.dumps(kats, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
