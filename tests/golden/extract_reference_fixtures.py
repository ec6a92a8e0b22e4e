#!/usr/bin/env python3
"""Write tests/golden/reference_fixtures.json from the reference's fixture data.

Reads the reference's hash-only fixtures for the MoE path
(fixtures/{router,expert,mixture,sparse_moe}/*.json under /root/reference) and
keeps the parts usable without the 360 GB checkpoint: input specifications,
input SHA-256s, selected experts, selected logits, normalised scores and the
mixture's score bits. Single-element captures (the shared-expert gate logit and
its sigmoid) are hashes of two bytes, so their bf16 values are recovered here by
exhaustive search over the 65,536 patterns and stored as values.

Run once in a container where /root/reference exists; the JSON it writes is
committed and the tests read only that.
"""
from __future__ import annotations

import hashlib
import json
import struct
from pathlib import Path

REFERENCE = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "reference_fixtures.json"


def recover_single_bf16(sha: str) -> int:
    for bits in range(65536):
        if hashlib.sha256(struct.pack("<H", bits)).hexdigest() == sha:
            return bits
    raise ValueError(f"no bf16 value hashes to {sha}")


def main() -> None:
    router = json.loads((REFERENCE / "fixtures/router/qwen3_8_flash_next_real.json").read_text())
    expert = json.loads((REFERENCE / "fixtures/expert/qwen3_8_flash_next_real.json").read_text())
    mixture = json.loads((REFERENCE / "fixtures/mixture/qwen3_8_flash_next_real.json").read_text())
    sparse = json.loads((REFERENCE / "fixtures/sparse_moe/qwen3_8_flash_next_layer0.json").read_text())
    out = {
        "source": "fixtures/{router,expert,mixture,sparse_moe} of the reference (hash-only, real checkpoint)",
        "router": {
            "configuration": router["configuration"],
            "cases": [
                {k: c[k] for k in ("name", "layer", "input_spec", "input_bf16_sha256",
                                   "selected_experts", "selected_logits_bf16",
                                   "normalized_scores_bf16")}
                for c in router["cases"]
            ],
        },
        "expert": {
            "configuration": expert["configuration"],
            "case": {k: expert["case"][k] for k in ("name", "layer", "expert", "route_weight_bf16",
                                                    "input_spec", "input_bf16_sha256")},
        },
        "mixture": {
            "case": {
                "top_k_selection_order": mixture["case"]["top_k_selection_order"],
                "expert_execution_order": mixture["case"]["expert_execution_order"],
                "route_weights_bf16": {str(e["expert"]): e["route_weight_bf16"]
                                       for e in mixture["case"]["experts"]},
                "input_bf16_sha256": mixture["case"]["input_bf16_sha256"],
            },
            # src/expert.rs:811-815
            "selection": [376, 349, 384, 191, 211, 363, 337, 206, 247, 295],
            "execution": [191, 206, 211, 247, 295, 337, 349, 363, 376, 384],
            "score_bits_by_selection": [0x3df5, 0x3de4, 0x3dd5, 0x3dd0, 0x3dca, 0x3dc5, 0x3dc3,
                                        0x3dc0, 0x3db8, 0x3db8],
        },
        "sparse_moe": {
            "input_spec": sparse["case"]["input_spec"],
            "input_bf16_sha256": sparse["case"]["input_bf16_sha256"],
            "shared_gate_logit_bits": recover_single_bf16(
                sparse["case"]["expected_bf16_sha256"]["shared_gate_logit"]),
            "shared_gate_sigmoid_bits": recover_single_bf16(
                sparse["case"]["expected_bf16_sha256"]["shared_gate_sigmoid"]),
        },
        # tests/test_generate_expert_fixture.py:29-35
        "capture_hash_bf16_one_minus_two":
            "7b429b1e3fd37fd03505ae4982471ea2c830392213b48a4e69976b5ebebce8e4",
    }
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
