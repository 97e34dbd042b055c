"""Writes tests/golden/parity_vectors.json from the reference's parity manifests.

Run in the build container (the reference is mounted at /root/reference):
    python tests/golden/make_fixtures.py

Each case pairs the inputs of a reference parity tool (a few literal
floats, transcribed with the tool's file:line) with the output bits its
manifest records (snapshots/parity/<family>/manifest.txt).  The JSON file is
data only; tests read it on any machine.
"""
from __future__ import annotations

import json
import re
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "parity_vectors.json"


def manifest(family: str) -> dict:
    path = REF / "snapshots" / "parity" / family / "manifest.txt"
    cases = {}
    for line in path.read_text().splitlines():
        m = re.match(r"case=(\S+) status=(\S+)(.*)", line)
        if not m:
            continue
        rest = m.group(3)
        bits = re.search(r"output_bits=([0-9a-f,]*)", rest)
        err = re.search(r"error=(\S+)", rest)
        cases[m.group(1)] = {
            "status": m.group(2),
            "error": err.group(1) if err else None,
            "output_bits": [int(b, 16) for b in bits.group(1).split(",") if b] if bits else [],
        }
    return {"source": str(path.relative_to(REF)), "cases": cases}


def main() -> None:
    fx = {}

    # tools/emel-kernel-binary-parity/src/main.rs:150-255
    b = manifest("kernel-binary")
    lhs, rhs = [1.0, 2.0, 3.0, 4.0], [10.0, 20.0, 30.0, 40.0]
    dense, dense_nb = [4, 1, 1, 1], [4, 16, 64, 64]
    fx["binary"] = {
        "source": b["source"],
        "inputs": "tools/emel-kernel-binary-parity/src/main.rs:150-255",
        "cases": [
            {"name": f"dense_{op}", "op": op, "lhs": lhs, "lhs_ne": dense, "lhs_nb": dense_nb, "rhs": rhs,
             "rhs_ne": dense, "rhs_nb": dense_nb, "out_len": 4, "out_fill": 0.0, "out_ne": dense, "out_nb": dense_nb,
             **b["cases"][f"dense_{op}"]}
            for op in ("add", "sub", "mul", "div")
        ] + [
            {"name": "strided_add", "op": "add", "lhs": [1.0, 99.0, 2.0, 99.0, 3.0], "lhs_ne": [3, 1, 1, 1],
             "lhs_nb": [8, 24, 72, 72], "rhs": [10.0, 99.0, 20.0, 99.0, 30.0], "rhs_ne": [3, 1, 1, 1],
             "rhs_nb": [8, 24, 72, 72], "out_len": 5, "out_fill": 0.0, "out_ne": [3, 1, 1, 1],
             "out_nb": [8, 24, 72, 72], **b["cases"]["strided_add"]},
            {"name": "count_equal_different_dimensions", "op": "add", "lhs": lhs, "lhs_ne": [2, 2, 1, 1],
             "lhs_nb": [4, 8, 16, 16], "rhs": rhs, "rhs_ne": dense, "rhs_nb": dense_nb, "out_len": 4,
             "out_fill": 0.0, "out_ne": dense, "out_nb": dense_nb,
             **b["cases"]["count_equal_different_dimensions"]},
            {"name": "implicit_contiguous_mul", "op": "mul", "lhs": lhs, "lhs_ne": dense, "lhs_nb": [0, 0, 0, 0],
             "rhs": rhs, "rhs_ne": dense, "rhs_nb": [0, 0, 0, 0], "out_len": 4, "out_fill": 0.0, "out_ne": dense,
             "out_nb": [0, 0, 0, 0], **b["cases"]["implicit_contiguous_mul"]},
            {"name": "count_mismatch_rejection", "op": "div", "lhs": lhs, "lhs_ne": dense, "lhs_nb": dense_nb,
             "rhs": rhs, "rhs_ne": dense, "rhs_nb": dense_nb, "out_len": 3, "out_fill": 9.0,
             "out_ne": [3, 1, 1, 1], "out_nb": [4, 12, 36, 36], **b["cases"]["count_mismatch_rejection"]},
        ],
    }

    # tools/emel-kernel-broadcast-parity/src/main.rs:50-95
    r = manifest("kernel-broadcast")
    fx["broadcast"] = {
        "source": r["source"],
        "inputs": "tools/emel-kernel-broadcast-parity/src/main.rs:50-95",
        "src0": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], "row": [10.0, 20.0, 30.0], "ne": [3, 2, 1, 1],
        "row_ne": [3, 1, 1, 1], "nb": [4, 12, 24, 24], "row_nb": [4, 12, 12, 12],
        "cases": [
            {"name": "row_add", "op": "add", "implicit": False, **r["cases"]["row_add"]},
            {"name": "row_mul", "op": "mul", "implicit": False, **r["cases"]["row_mul"]},
            {"name": "row_add_implicit", "op": "add", "implicit": True, **r["cases"]["row_add_implicit"]},
        ],
    }

    # tools/emel-kernel-softmax-parity/src/main.rs:23-80
    s = manifest("kernel-softmax")
    fx["softmax"] = {
        "source": s["source"],
        "inputs": "tools/emel-kernel-softmax-parity/src/main.rs:23-80",
        "input": [1.0, 2.0, 4.0, 2.0, 5.0, 8.0], "ne": [3, 2, 1, 1],
        "cases": s["cases"],
        "sentinel_bits": 0x7FC00001,
    }

    # tools/emel-kernel-normalization-parity/src/main.rs:37-105
    n = manifest("kernel-normalization")
    fx["normalization"] = {
        "source": n["source"],
        "inputs": "tools/emel-kernel-normalization-parity/src/main.rs:37-105",
        "rms_input": [1.0, 2.0, 4.0, 2.0, 5.0, 8.0], "rms_ne": [3, 2, 1, 1], "rms_nb": [0, 0, 0, 0],
        "norm_input": [1.0, 2.0, 99.0, 99.0, 2.0, 5.0, 8.0], "norm_ne": [3, 2, 1, 1], "norm_nb": [4, 16, 32, 32],
        "epsilon": 1.0,
        "cases": n["cases"],
    }

    # tools/emel-kernel-unary-parity/src/main.rs:25-60; the manifest compares
    # libm-backed ops with a four-ULP tolerance (manifest lines 23, 26).
    u = manifest("kernel-unary")
    fx["unary"] = {
        "source": u["source"],
        "inputs": "tools/emel-kernel-unary-parity/src/main.rs:25",
        "input": [-10.1, -10.0, -1.2345, -0.125, 0.0, 0.12345, 10.0, 10.1],
        "subops": {"abs": 0, "neg": 2, "relu": 6, "exp": 13, "tanh": 4, "elu": 5, "gelu": 8, "silu": 10},
        "libm_ulp_tolerance": 4,
        "libm_ops": ["exp", "tanh", "elu", "silu"],
        "cases": u["cases"],
    }

    # tools/emel-kernel-elementwise-parity/src/main.rs:69-125
    e = manifest("kernel-elementwise")
    fx["elementwise"] = {
        "source": e["source"],
        "inputs": "tools/emel-kernel-elementwise-parity/src/main.rs:69-125",
        "input": [1.5, -2.0, 0.25], "other": [-0.5, 4.0, 2.0],
        "cases": {k: v for k, v in e["cases"].items() if k in ("op_add", "op_sub", "op_mul", "op_div")},
    }

    # tools/emel-kernel-activation-parity/src/main.rs:42-55
    a = manifest("kernel-activation")
    fx["activation"] = {
        "source": a["source"],
        "inputs": "tools/emel-kernel-activation-parity/src/main.rs:42-55",
        "input_bits": [0xC0000000, 0xBF000000, 0x00000000, 0x40000000, 0x7FC01234],
        "scale": 1.5,
        "cases": {"op_scale": a["cases"]["op_scale"]},
    }

    # Known-answer unit tests (crates/emel-kernels/tests/any/).
    fx["known_answers"] = {
        "reductions": {
            "source": "crates/emel-kernels/tests/any/reductions.rs:58-102",
            "input": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], "ne": [3, 2, 1, 1],
            "sum": 21.0, "mean": 3.5, "argmax": 5.0, "sum_rows": [6.0, 15.0],
        },
        "rms_norm": {
            "source": "crates/emel-kernels/tests/any/normalization_ops.rs:57-73",
            "input": [3.0, 4.0, 0.0, 2.0], "ne": [2, 2, 1, 1], "epsilon": 1.0,
            "output": [0.8164966, 1.0886621, 0.0, 1.1547005],
        },
        "silu": {
            "source": "crates/emel-kernels/tests/any/unary_ops.rs:23-77",
            "input": [-2.0, -0.5, 0.5, 2.0], "index": 2, "value": 0.31122968, "abs_tol": 1e-6,
        },
        "softmax_stability": {
            "source": "crates/emel-kernels/tests/any/reductions.rs:105-122",
            "input": [1000.0, 1001.0, 1002.0, -1000.0, -999.0, -998.0], "ne": [3, 2, 1, 1], "row_sum_tol": 1e-6,
        },
    }

    # tools/emel-kernel-power-parity/src/main.rs:118-155 (root slice events
    # and the view PowerKernel)
    pw = manifest("kernel-power")
    fx["power"] = {
        "source": pw["source"],
        "inputs": "tools/emel-kernel-power-parity/src/main.rs:118-155",
        "cases": [
            {"name": "dense_square", "route": "slice_sqr", "input": [-2.0, -0.5, 0.5, 2.0], "out_len": 4,
             "out_fill": 0.0, **pw["cases"]["dense_square"]},
            {"name": "strided_square", "route": "view_sqr", "input": [3.0, 99.0, -4.0, 99.0, 0.5], "ne": [3, 1, 1, 1],
             "nb": [8, 24, 72, 72], "out_len": 5, "out_fill": 0.0, **pw["cases"]["strided_square"]},
            {"name": "count_equal_different_dimensions", "route": "slice_sqr", "input": [1.0, 2.0, 3.0, 4.0],
             "out_len": 4, "out_fill": 0.0, **pw["cases"]["count_equal_different_dimensions"]},
            {"name": "implicit_contiguous_square", "route": "view_sqr", "input": [1.0, 2.0, 3.0, 4.0],
             "ne": [4, 1, 1, 1], "nb": [0, 0, 0, 0], "out_len": 4, "out_fill": 0.0,
             **pw["cases"]["implicit_contiguous_square"]},
            {"name": "dense_square_root", "route": "slice_sqrt", "input": [0.0, 1.0, 4.0, 9.0], "out_len": 4,
             "out_fill": 0.0, **pw["cases"]["dense_square_root"]},
            {"name": "shape_rejection", "route": "slice_sqr", "input": [1.0, 2.0, 3.0, 4.0], "out_len": 3,
             "out_fill": 9.0, **pw["cases"]["shape_rejection"]},
        ],
    }
    # crates/emel-kernels/tests/any/ops.rs:13-124 (root dense-slice events)
    fx["known_answers"]["slice_ops"] = {
        "source": "crates/emel-kernels/tests/any/ops.rs:13-124",
        "dup": {"input": [1.0, -2.5, 4.0], "output": [1.0, -2.5, 4.0]},
        "add": {"lhs": [1.0, -2.5, 4.0], "rhs": [2.0, 0.5, -1.0], "output": [3.0, -2.0, 3.0]},
        "sub": {"lhs": [9.0, -4.0, 2.0], "rhs": [3.0, 2.0, -4.0], "output": [6.0, -6.0, 6.0]},
        "mul": {"lhs": [9.0, -4.0, 2.0], "rhs": [3.0, 2.0, -4.0], "output": [27.0, -8.0, -8.0]},
        "div": {"lhs": [9.0, -4.0, 2.0], "rhs": [3.0, 2.0, -4.0], "output": [3.0, -2.0, -0.5]},
        "sqr": {"input": [3.0, 2.0, -4.0], "output": [9.0, 4.0, 16.0]},
        "sqrt": {"input": [9.0, 4.0, 16.0], "output": [3.0, 2.0, 4.0]},
        "invalid_shape": [
            {"event": "dup", "in_len": 2, "out_len": 1}, {"event": "add", "lhs_len": 2, "rhs_len": 1, "out_len": 2},
            {"event": "dup", "in_len": 0, "out_len": 0}, {"event": "sub", "lhs_len": 2, "rhs_len": 1, "out_len": 2},
            {"event": "mul", "lhs_len": 2, "rhs_len": 1, "out_len": 2},
            {"event": "div", "lhs_len": 2, "rhs_len": 1, "out_len": 2},
            {"event": "sqr", "in_len": 2, "out_len": 1}, {"event": "sqrt", "in_len": 2, "out_len": 1},
        ],
    }

    OUT.write_text(json.dumps(fx, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
