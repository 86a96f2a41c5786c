"""The oracle and the host logic against the committed golden fixtures
(tests/golden/, written by tests/golden/make_golden.py).  No GPU work."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
import qmm as Q

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return json.loads((GOLDEN / name).read_text())


@pytest.mark.parametrize("mode", ["mxfp8", "nvfp4"])
def test_oracle_reproduces_reference_qmm_case(mode):
    """src/model.zig:1561-1609: quantize, dequantize and qmm of the reference's integer case."""
    g = load("reference_qmm_case.json")
    W = np.array(g["W"], np.float32)
    x = np.array(g["x"], np.float32)
    y = np.array(g["y"], np.float32)
    gm = g["modes"][mode]
    wq, s = O.quantize(mode, W)
    assert np.array_equal(wq, np.array(gm["w"], np.uint32))
    assert np.array_equal(s, np.array(gm["scales"], np.uint8))
    assert np.array_equal(O.dequant(mode, wq, s, 32), W)
    assert np.array_equal(O.qmm(mode, x, wq, s, x_is_bf16=False, out="f32"), y)
    assert np.array_equal(O.bf16_bits_to_f32(O.qmm(mode, O.f32_to_bf16_bits(x), wq, s)), y)


def test_infer_quant_spec_golden_cases():
    """src/weights.zig:493-541 headers, replayed against the C++ loader's inference."""
    g = load("infer_quant_spec_cases.json")
    assert len(g["cases"]) == 5
    for case in g["cases"]:
        got = Q.infer_quant_spec_json(case["header"])
        exp = case["expect"]
        if "error" in exp:
            assert got == exp["error"], case
        elif exp["mode"] == "none":
            assert got[0] == "none", case
        else:
            assert got == (exp["mode"], exp["group"], exp["bits"]), case
