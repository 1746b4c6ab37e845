#!/usr/bin/env python3
"""Writes reference_kats.json: the known-answer vectors that the reference's own
tests state literally (inputs and exact expected outputs), transcribed as data
with the file:line each comes from.  Run from anywhere:

    python tests/golden/make_golden.py

The reference is Rust and is not built here; these vectors are what its tests
assert, so a mismatch against them is a mismatch against the reference.
"""
import json
from pathlib import Path

KATS = [
    {
        "name": "add_in_place",
        "source": "src/cuda.rs:1376-1379 (driver_round_trip_preserves_f32_values_when_explicitly_enabled)",
        "op": "add",
        "dst": [1.0, -2.0, 3.5],
        "src": [0.5, 2.0, -1.0],
        "expected": [1.5, 0.0, 2.5],
    },
    {
        "name": "overwrite_prefix_and_segments",
        "source": "src/cuda.rs:1381-1400",
        "op": "copy_ops",
        "source_values": [9.0, 8.0, 7.0, 6.0],
        "replacement": [-1.0, -2.0],
        "after_overwrite_prefix_2": [-1.0, -2.0, 7.0, 6.0],
        "segment_1_2": [8.0, 7.0],
        "after_copy_segment_into_2": [-1.0, -2.0, 8.0, 7.0],
    },
    {
        "name": "gemm_row_major_2x3x2",
        "source": "src/cuda.rs:1402-1411",
        "op": "gemm",
        "m": 2, "k": 3, "n": 2,
        "a": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
        "b": [7.0, 8.0, 9.0, 10.0, 11.0, 12.0],
        "expected": [58.0, 64.0, 139.0, 154.0],
    },
    {
        "name": "bias_scale_2x2",
        "source": "src/cuda.rs:1413-1422",
        "op": "bias_scale",
        "rows": 2, "cols": 2,
        "values": [58.0, 64.0, 139.0, 154.0],
        "bias": [1.0, -4.0],
        "gamma": [0.5, 2.0],
        "expected": [29.5, 120.0, 70.0, 300.0],
    },
    {
        "name": "chained_linear_and_run_chw",
        "source": "src/cuda.rs:1435-1461",
        "op": "linear_chain",
        "input": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], "rows": 2,
        "first": {"in": 3, "out": 2, "w": [7.0, 8.0, 9.0, 10.0, 11.0, 12.0], "b": [1.0, -4.0], "gamma": [0.5, 2.0]},
        "second": {"in": 2, "out": 1, "w": [2.0, -1.0], "b": [3.0], "gamma": None},
        "expected_chain": [-58.0, -157.0],
        "expected_first_chw": [29.5, 70.0, 120.0, 300.0],
    },
    {
        "name": "gemm_2x2_identity",
        "source": "tests/scalar_ops.rs:3-10",
        "op": "gemm",
        "m": 2, "k": 2, "n": 2,
        "a": [1.0, 2.0, 3.0, 4.0],
        "b": [1.0, 0.0, 0.0, 1.0],
        "expected": [1.0, 2.0, 3.0, 4.0],
    },
    {
        "name": "layerscale_2x3",
        "source": "tests/scalar_ops.rs:42-49",
        "op": "layerscale",
        "rows": 2, "cols": 3,
        "values": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
        "gamma": [10.0, -1.0, 0.5],
        "expected": [10.0, -2.0, 1.5, 40.0, -5.0, 3.0],
    },
    {
        "name": "gelu_zero_and_large",
        "source": "tests/scalar_ops.rs:22-29",
        "op": "gelu_bounds",
        "values": [0.0, 10.0, -10.0],
        "bounds": [[0.0, 1e-6], [10.0, 1e-3], [0.0, 1e-3]],
    },
    {
        "name": "softmax_rows",
        "source": "tests/scalar_ops.rs:12-20",
        "op": "softmax_bounds",
        "rows": 2, "cols": 3,
        "values": [1.0, 2.0, 3.0, 0.0, 0.0, 0.0],
        "row_sum": 1.0, "tol": 1e-6,
        "uniform_row": 1, "uniform_value": 1.0 / 3.0,
    },
]


def main() -> None:
    out = Path(__file__).resolve().parent / "reference_kats.json"
    out.write_text(json.dumps({"kats": KATS}, indent=1) + "\n")
    print(f"wrote {out} ({len(KATS)} vectors)")


if __name__ == "__main__":
    main()
