"""The reference's literal known-answer vectors (tests/golden/reference_kats.json,
written by tests/golden/make_golden.py with the file:line of each) checked
against the CPU oracle and, through the C ABI, against the HIP path."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O

KATS = {k["name"]: k for k in json.loads(
    (Path(__file__).resolve().parent / "golden" / "reference_kats.json").read_text())["kats"]}


def f32(v):
    return np.asarray(v, dtype=np.float32)


def exact(got, expected):
    assert np.array_equal(f32(got), f32(expected)), (got, expected)


# ---- oracle ---------------------------------------------------------------------

def test_fixture_is_current():
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "make_golden", Path(__file__).resolve().parent / "golden" / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert [k["name"] for k in mod.KATS] == list(KATS)
    assert json.loads(json.dumps({"kats": mod.KATS})) == {"kats": list(KATS.values())}


def test_oracle_add():
    k = KATS["add_in_place"]
    exact(O.add(f32(k["dst"]), f32(k["src"])), k["expected"])


@pytest.mark.parametrize("name", ["gemm_row_major_2x3x2", "gemm_2x2_identity"])
def test_oracle_gemm(name):
    k = KATS[name]
    exact(O.gemm_f32(f32(k["a"]), f32(k["b"]), k["m"], k["n"], k["k"]), k["expected"])
    exact(O.linear(f32(k["a"]), f32(k["b"]), k["m"], k["n"], k["k"]), k["expected"])


def test_oracle_bias_scale_and_layerscale():
    k = KATS["bias_scale_2x2"]
    v = O.add_bias_rows(f32(k["values"]), k["rows"], k["cols"], f32(k["bias"]))
    exact(O.layerscale(v, k["rows"], k["cols"], f32(k["gamma"])), k["expected"])
    k = KATS["layerscale_2x3"]
    exact(O.layerscale(f32(k["values"]), k["rows"], k["cols"], f32(k["gamma"])), k["expected"])


def test_oracle_linear_chain():
    k = KATS["chained_linear_and_run_chw"]
    a, f, s = f32(k["input"]), k["first"], k["second"]
    h = O.linear_bias_scale(a, f32(f["w"]), f32(f["b"]), f32(f["gamma"]), k["rows"], f["out"], f["in"])
    exact(h.reshape(k["rows"], f["out"]).T.reshape(-1), k["expected_first_chw"])
    y = O.add_bias_rows(O.linear(h, f32(s["w"]), k["rows"], s["out"], s["in"]), k["rows"], s["out"],
                        f32(s["b"]))
    exact(y, k["expected_chain"])


def test_oracle_gelu_and_softmax_bounds():
    k = KATS["gelu_zero_and_large"]
    got = O.gelu(f32(k["values"]))
    for g, (target, tol) in zip(got, k["bounds"]):
        assert abs(g - target) < tol
    k = KATS["softmax_rows"]
    got = O.softmax_rows(f32(k["values"]), k["rows"], k["cols"]).reshape(k["rows"], k["cols"])
    assert np.all(np.abs(got.sum(axis=1) - k["row_sum"]) < k["tol"])
    assert abs(got[k["uniform_row"], 0] - k["uniform_value"]) < k["tol"]


# ---- HIP path through the C ABI --------------------------------------------------

@pytest.mark.gpu
def test_gpu_reference_kats(rt):
    k = KATS["add_in_place"]
    t = rt.upload_f32(f32(k["dst"]))
    rt.add_f32_in_place(t, rt.upload_f32(f32(k["src"])))
    exact(rt.download_f32(t), k["expected"])

    k = KATS["overwrite_prefix_and_segments"]
    src = rt.upload_f32(f32(k["source_values"]))
    copied = rt.copy_f32(src)
    rt.overwrite_prefix_f32(copied, rt.upload_f32(f32(k["replacement"])), 2)
    exact(rt.download_f32(copied), k["after_overwrite_prefix_2"])
    seg = rt.copy_segment_f32(src, 1, 2)
    exact(rt.download_f32(seg), k["segment_1_2"])
    rt.copy_segment_into_f32(copied, 2, seg, 0, 2)
    exact(rt.download_f32(copied), k["after_copy_segment_into_2"])

    for name in ("gemm_row_major_2x3x2", "gemm_2x2_identity"):
        k = KATS[name]
        c = rt.gemm_row_major_f32(rt.upload_f32(f32(k["a"])), rt.upload_f32(f32(k["b"])), k["m"],
                                  k["k"], k["n"])
        exact(rt.download_f32(c), k["expected"])

    k = KATS["bias_scale_2x2"]
    v = rt.upload_f32(f32(k["values"]))
    rt.bias_scale_f32_in_place(v, rt.upload_f32(f32(k["bias"])), rt.upload_f32(f32(k["gamma"])),
                               k["rows"], k["cols"])
    exact(rt.download_f32(v), k["expected"])

    k = KATS["chained_linear_and_run_chw"]
    f, s = k["first"], k["second"]
    first = rt.prepare_linear_f32(f["in"], f["out"], f32(f["w"]), f32(f["b"]), f32(f["gamma"]))
    second = rt.prepare_linear_f32(s["in"], s["out"], f32(s["w"]), f32(s["b"]), None)
    a = rt.upload_f32(f32(k["input"]))
    exact(rt.download_f32(second.run(first.run(a, k["rows"]), k["rows"])), k["expected_chain"])
    exact(rt.download_f32(first.run_chw(a, k["rows"])), k["expected_first_chw"])

    k = KATS["gelu_zero_and_large"]
    g = rt.upload_f32(f32(k["values"]))
    rt.gelu_f32_in_place(g)
    for v, (target, tol) in zip(rt.download_f32(g), k["bounds"]):
        assert abs(v - target) < tol
