"""Pins the CPU oracle to the reference's own golden vectors.

Expected bits come from the reference's parity manifests
(snapshots/parity/*/manifest.txt) and known-answer unit tests
(crates/emel-kernels/tests/any/*.rs), collected into
tests/golden/parity_vectors.json by tests/golden/make_fixtures.py.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as orc
from helpers import bits, ulp_distance

FX = json.loads((Path(__file__).parent / "golden" / "parity_vectors.json").read_text())
OPS = {"add": orc.ADD, "sub": orc.SUB, "mul": orc.MUL, "div": orc.DIV}


def logical(buf, ne, nb):
    """Logical-ordinal read-back, as the parity tools print outputs."""
    if nb[0] == 0:
        nb = [4, 4 * ne[0], 4 * ne[0] * ne[1], 4 * ne[0] * ne[1] * ne[2]]
    out = []
    for k in range(int(np.prod(ne))):
        rem, off = k, 0
        for d in range(4):
            off += (rem % ne[d]) * nb[d]
            rem //= ne[d]
        out.append(buf[off // 4])
    return np.array(out, dtype=np.float32)


@pytest.mark.parametrize("case", FX["binary"]["cases"], ids=lambda c: c["name"])
def test_binary_manifest(case):
    lhs = np.array(case["lhs"], np.float32)
    rhs = np.array(case["rhs"], np.float32)
    out = np.full(case["out_len"], case["out_fill"], np.float32)
    st = orc.binary(OPS[case["op"]], orc.view(lhs, case["lhs_ne"], case["lhs_nb"]),
                    orc.view(rhs, case["rhs_ne"], case["rhs_nb"]), orc.view(out, case["out_ne"], case["out_nb"]))
    assert (st == orc.OK) == (case["status"] == "ok")
    if case["status"] != "ok":
        assert st == orc.SHAPE_MISMATCH
    got = logical(out, case["out_ne"], case["out_nb"])
    assert list(bits(got)) == case["output_bits"]


@pytest.mark.parametrize("case", FX["broadcast"]["cases"], ids=lambda c: c["name"])
def test_broadcast_manifest(case):
    fx = FX["broadcast"]
    src0 = np.array(fx["src0"], np.float32)
    row = np.array(fx["row"], np.float32)
    out = np.zeros(6, np.float32)
    nb = [0, 0, 0, 0] if case["implicit"] else fx["nb"]
    rnb = [0, 0, 0, 0] if case["implicit"] else fx["row_nb"]
    st = orc.broadcast_row(OPS[case["op"]], orc.view(src0, fx["ne"], nb), orc.view(row, fx["row_ne"], rnb),
                           orc.view(out, fx["ne"], nb))
    assert st == orc.OK
    assert list(bits(logical(out, fx["ne"], nb))) == case["output_bits"]


def test_softmax_manifest():
    fx = FX["softmax"]
    x = np.array(fx["input"], np.float32)
    for name, nb in (("dense_rows", None), ("implicit_contiguous", [0, 0, 0, 0])):
        out = np.zeros(6, np.float32)
        assert orc.soft_max(orc.view(x, fx["ne"], nb), orc.view(out, fx["ne"], nb)) == orc.OK
        assert list(bits(out)) == fx["cases"][name]["output_bits"], name
    sentinel = np.full(4, np.uint32(fx["sentinel_bits"]).view(np.float32), np.float32)
    assert orc.soft_max(orc.view(x, fx["ne"]), orc.view(sentinel, [2, 2, 1, 1])) == orc.SHAPE_MISMATCH
    assert list(bits(sentinel)) == fx["cases"]["shape_mismatch"]["output_bits"]
    # invalid dtype (F16 with F32 strides, tools/emel-kernel-softmax-parity/src/main.rs:51-63)
    typed = np.full(6, np.uint32(fx["sentinel_bits"]).view(np.float32), np.float32)
    assert orc.soft_max(orc.view(x, fx["ne"], None, orc.F16), orc.view(typed, fx["ne"], None, orc.F16)) == orc.INVALID_VIEW
    assert (bits(typed) == fx["sentinel_bits"]).all()


def test_normalization_manifest():
    fx = FX["normalization"]
    x = np.array(fx["rms_input"], np.float32)
    out = np.zeros(6, np.float32)
    assert orc.rms_norm(orc.view(x, fx["rms_ne"], fx["rms_nb"]), orc.view(out, fx["rms_ne"], fx["rms_nb"]), 1.0) == orc.OK
    assert list(bits(out)) == fx["cases"]["implicit_rms_norm"]["output_bits"]

    xs = np.array(fx["norm_input"], np.float32)
    out = np.full(7, 9.0, np.float32)
    assert orc.norm(orc.view(xs, fx["norm_ne"], fx["norm_nb"]), orc.view(out, fx["norm_ne"], fx["norm_nb"]), 1.0) == orc.OK
    assert list(bits(out)) == fx["cases"]["strided_norm"]["output_bits"]

    one = np.array([1.0], np.float32)
    out = np.full(1, 9.0, np.float32)
    assert orc.norm(orc.view(one, [3, 0, 1, 1], [4, 12, 0, 0]), orc.view(out, [3, 0, 1, 1], [4, 12, 0, 0]), 1.0) == orc.INVALID_VIEW
    assert list(bits(out)) == fx["cases"]["empty_outer_norm"]["output_bits"]

    out = np.full(6, 9.0, np.float32)
    st = orc.norm(orc.view(x, fx["rms_ne"], fx["rms_nb"]), orc.view(out, fx["rms_ne"], fx["rms_nb"]), float("nan"))
    assert st == orc.INVALID_PARAMETERS
    assert list(bits(out)) == fx["cases"]["invalid_epsilon"]["output_bits"]


@pytest.mark.parametrize("name", list(FX["unary"]["subops"]))
def test_unary_manifest(name):
    fx = FX["unary"]
    x = np.array(fx["input"], np.float32)
    out = np.zeros(8, np.float32)
    assert orc.unary(fx["subops"][name], orc.view(x, [8, 1, 1, 1], [4, 32, 32, 32]),
                     orc.view(out, [8, 1, 1, 1], [4, 32, 32, 32])) == orc.OK
    want = np.array(fx["cases"][name]["output_bits"], np.uint32).view(np.float32)
    if name in fx["libm_ops"]:
        # The manifest itself compares libm-backed results within 4 ULP.
        assert ulp_distance(out, want).max() <= fx["libm_ulp_tolerance"]
    else:
        assert list(bits(out)) == fx["cases"][name]["output_bits"]


def test_elementwise_manifest():
    fx = FX["elementwise"]
    a = np.array(fx["input"], np.float32)
    b = np.array(fx["other"], np.float32)
    for name, op in (("op_add", orc.ADD), ("op_sub", orc.SUB), ("op_mul", orc.MUL), ("op_div", orc.DIV)):
        out = np.zeros(3, np.float32)
        assert orc.binary(op, orc.view(a, [3, 1, 1, 1]), orc.view(b, [3, 1, 1, 1]), orc.view(out, [3, 1, 1, 1])) == orc.OK
        assert list(bits(out)) == fx["cases"][name]["output_bits"], name


def test_scale_manifest():
    fx = FX["activation"]
    x = np.array(fx["input_bits"], np.uint32).view(np.float32).copy()
    out = np.zeros(5, np.float32)
    assert orc.scale(orc.view(x, [5, 1, 1, 1]), orc.view(out, [5, 1, 1, 1]), fx["scale"]) == orc.OK
    assert list(bits(out)) == fx["cases"]["op_scale"]["output_bits"]


def test_reduction_known_answers():
    k = FX["known_answers"]["reductions"]
    x = np.array(k["input"], np.float32)
    s = np.zeros(1, np.float32)
    assert orc.sum_(orc.view(x, k["ne"]), orc.view(s, [1, 1, 1, 1])) == orc.OK and s[0] == k["sum"]
    assert orc.mean(orc.view(x, k["ne"]), orc.view(s, [1, 1, 1, 1])) == orc.OK and s[0] == k["mean"]
    assert orc.argmax(orc.view(x, k["ne"]), orc.view(s, [1, 1, 1, 1])) == orc.OK and s[0] == k["argmax"]
    rows = np.zeros(2, np.float32)
    assert orc.sum_rows(orc.view(x, k["ne"]), orc.view(rows, [1, 2, 1, 1])) == orc.OK
    assert list(rows) == k["sum_rows"]


def test_rms_norm_known_answer():
    k = FX["known_answers"]["rms_norm"]
    x = np.array(k["input"], np.float32)
    out = np.zeros(4, np.float32)
    assert orc.rms_norm(orc.view(x, k["ne"]), orc.view(out, k["ne"]), k["epsilon"]) == orc.OK
    assert list(bits(out)) == list(bits(np.array(k["output"], np.float32)))


def test_silu_known_answer():
    k = FX["known_answers"]["silu"]
    x = np.array(k["input"], np.float32)
    out = np.zeros(4, np.float32)
    assert orc.unary_event(10, orc.view(x, [4, 1, 1, 1]), orc.view(out, [4, 1, 1, 1])) == orc.OK
    assert abs(out[k["index"]] - k["value"]) < k["abs_tol"]


def test_softmax_stability_known_answer():
    k = FX["known_answers"]["softmax_stability"]
    x = np.array(k["input"], np.float32)
    out = np.zeros(6, np.float32)
    assert orc.soft_max(orc.view(x, k["ne"]), orc.view(out, k["ne"])) == orc.OK
    assert np.isfinite(out).all()
    assert abs(out[:3].sum() - 1.0) < k["row_sum_tol"] and abs(out[3:].sum() - 1.0) < k["row_sum_tol"]


@pytest.mark.parametrize("case", FX["power"]["cases"], ids=lambda c: c["name"])
def test_power_manifest(case):
    """snapshots/parity/kernel-power: root OpSqr/OpSqrt over slices and the
    view PowerKernel (strided and implicit layouts)."""
    inp = np.array(case["input"], np.float32)
    out = np.full(case["out_len"], case["out_fill"], np.float32)
    if case["route"] == "view_sqr":
        st = orc.op_power(False, orc.view(inp, case["ne"], case["nb"]), orc.view(out, case["ne"], case["nb"]))
        got = logical(out, case["ne"], case["nb"])
    else:
        st = orc.slice_power(case["route"] == "slice_sqrt", inp, out)
        got = out
    assert (st == orc.OK) == (case["status"] == "ok")
    if case["status"] != "ok":
        assert st == orc.INVALID_SHAPE
    assert list(bits(got)) == case["output_bits"]


def test_slice_ops_known_answers():
    """crates/emel-kernels/tests/any/ops.rs: root dense-slice events."""
    ka = FX["known_answers"]["slice_ops"]
    f = lambda xs: np.array(xs, np.float32)  # noqa: E731
    out = np.zeros(3, np.float32)
    assert orc.slice_dup(f(ka["dup"]["input"]), out) == orc.OK and list(out) == ka["dup"]["output"]
    for name, op in (("add", orc.ADD), ("sub", orc.SUB), ("mul", orc.MUL), ("div", orc.DIV)):
        c = ka[name]
        assert orc.slice_binary(op, f(c["lhs"]), f(c["rhs"]), out) == orc.OK
        assert list(out) == c["output"], name
    assert orc.slice_power(False, f(ka["sqr"]["input"]), out) == orc.OK and list(out) == ka["sqr"]["output"]
    assert orc.slice_power(True, f(ka["sqrt"]["input"]), out) == orc.OK and list(out) == ka["sqrt"]["output"]
    for case in ka["invalid_shape"]:
        ev = case["event"]
        if ev == "dup":
            st = orc.slice_dup(np.ones(max(case["in_len"], 1), np.float32), np.ones(max(case["out_len"], 1), np.float32),
                               case["in_len"], case["out_len"])
        elif ev in ("sqr", "sqrt"):
            st = orc.slice_power(ev == "sqrt", np.ones(case["in_len"], np.float32), np.ones(case["out_len"], np.float32))
        else:
            st = orc.slice_binary(OPS[ev], np.ones(case["lhs_len"], np.float32), np.ones(case["rhs_len"], np.float32),
                                  np.ones(case["out_len"], np.float32))
        assert st == orc.INVALID_SHAPE, case
