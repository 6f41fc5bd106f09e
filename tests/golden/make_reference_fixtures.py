"""Write ``reference_fixtures.json``: known answers transcribed from the
reference's own tests (values only; no reference code is imported or run).

Sources (file:line in the reference tree):
  tests/unit/test_quant_compute.py:14-23   AWQ pack order of values 0..7
  tests/unit/test_quant_compute.py:25-31   GPTQ LSB-first row packing
  tests/unit/test_quant_compute.py:62-68   FP8 clamp-before-cast of +-1000
  tests/unit/test_moe_precision.py:15-33   fixed router logits, top_k=2
  tests/unit/test_moe_precision.py:118-137 tie-break logits [1,1,1,0]
  tests/unit/test_moe_precision.py:138-154 fp32 combine before the bf16 cast
  tests/unit/test_moe_precision.py:194-226 slot-order combine of 4 slots
  tests/gpu/test_quant_kernels.py:42-69,116-227 kernel parity cases/tolerances

Run:  python tests/golden/make_reference_fixtures.py
"""

from __future__ import annotations

import json
from pathlib import Path

FIXTURES = {
    "awq_pack_order": {"values": list(range(8)), "nibbles": [0, 2, 4, 6, 1, 3, 5, 7]},
    "gptq_row_pack": {"values": list(range(8)), "nibbles": [0, 1, 2, 3, 4, 5, 6, 7]},
    "gptq_zero_offset_roundtrip": {"seed": 0, "shape": [16, 16], "group_size": 8, "max_err": 0.2},
    "fp8_clamp_before_cast": {"weight": [[1000.0, -1000.0]], "max_rel_err": 0.05},
    "fp8_roundtrip": {"seed": 1, "shape": [8, 32], "max_abs_err": 0.15},
    "awq_roundtrip": {"seed": 3, "shape": [16, 32], "group_size": 16, "max_abs_err": 0.3},
    "router_fixed": {
        "logits": [1.25, -0.5, 0.75, 0.125],
        "top_k": 2,
        "expected_indices": [0, 2],
    },
    "router_ties": {"logits": [1.0, 1.0, 1.0, 0.0], "top_k": 2, "expected_indices": [0, 1]},
    "combine_fp32_before_cast": {
        "expert_values": [-5.84375, -7.5625],
        "weights": [0.5715058445930481, 0.4284941852092743],
    },
    "combine_slot_order": {
        "expert_values": [0.66015625, 0.061767578125, 0.267578125, 0.62109375],
        "weights": [0.2010020762681961, 0.2674923539161682, 0.06888598203659058,
                    0.4626196026802063],
        "ep2_owner_slots": [[0, 2], [1, 3]],
    },
    "int8_act_quant_cases": {"seed": 356, "rows": 4, "k_sizes": [1536, 8960], "zero_row": 0},
    "int8_bitexact_cases": [
        {"k": 64, "seed": 1174, "n": 128, "m": 4},
        {"k": 1536, "seed": 357, "n": 128, "m": 4},
        {"k": 8960, "seed": 357, "n": 128, "m": 4},
    ],
    "ragged_shapes": [[1, 64, 32], [17, 96, 40], [32, 64, 32]],
    "tolerances": {
        "int8": {"rtol": 0.03, "atol": 0.08},
        "awq": {"rtol": 0.03, "atol": 0.08},
        "gptq": {"rtol": 0.03, "atol": 0.08},
        "fp8": {"rel_rmse": 0.035, "max_abs_per_sqrt_k": 0.12},
    },
    "w4a16_scale_precision": {"scale": 1.00390625, "rows": 3, "k": 64, "n": 32},
    "w4a16_saturation": {"value": 70000.0, "scale": 0.5, "rows": 3, "k": 64, "n": 32},
}


def main() -> None:
    path = Path(__file__).with_name("reference_fixtures.json")
    path.write_text(json.dumps(FIXTURES, indent=1, sort_keys=True) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
