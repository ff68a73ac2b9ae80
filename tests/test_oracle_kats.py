"""The reference's own known-answer tests (tests/test_reference.c:32-468),
restated as JSON data, run against the oracle restatement and, where it was
built, against the compiled reference (oracle/_ref)."""
import json
from pathlib import Path

import numpy as np
import pytest

import _oracle as O

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
EPS = KATS["eps"]


def backends():
    out = [("oracle", O.orc())]
    if O.ref() is not None:
        out.append(("reference", O.ref()))
    return out


@pytest.mark.parametrize("which", ["oracle", "reference"])
def test_rms_norm_softmax_silu_topk(which):
    libs = dict(backends())
    if which not in libs:
        pytest.skip("reference library not built")
    lib = libs[which]
    pre = "orc_" if which == "oracle" else "ds3_ref_"
    x = np.array(KATS["rms_norm"]["x"], np.float32)
    for case in KATS["rms_norm"]["cases"]:
        out = np.empty(4, np.float32)
        w = np.array(case["w"], np.float32)
        getattr(lib, pre + "rms_norm")(O.ptr(x), O.ptr(w), case["eps"], 4, O.ptr(out))
        for i, v in case["expect"].items():
            assert abs(out[int(i)] - v) <= EPS
    for case in KATS["softmax"]:
        v = np.array(case["x"], np.float32)
        getattr(lib, pre + "softmax")(O.ptr(v), v.size)
        assert abs(v.sum() - case["sum"]) <= EPS
        for i, e in case["expect"].items():
            assert abs(v[int(i)] - e) <= EPS
    s = KATS["silu"]
    xs = np.array(s["x"], np.float32)
    out = np.empty(3, np.float32)
    getattr(lib, pre + "silu")(O.ptr(xs), O.ptr(out), 3)
    assert np.all(np.abs(out - np.array(s["expect"], np.float32)) <= EPS)
    tk = KATS["topk"]
    sc = np.array(tk["scores"], np.float32)
    idx = np.empty(tk["k"], np.int32)
    val = np.empty(tk["k"], np.float32)
    getattr(lib, pre + "topk")(O.ptr(sc), sc.size, tk["k"], O.ptr(idx), O.ptr(val))
    assert idx.tolist() == tk["idx"]
    assert np.all(np.abs(val - np.array(tk["val"], np.float32)) <= EPS)


@pytest.mark.parametrize("case", KATS["dequant"], ids=lambda c: f"type{c['type']}")
def test_dequant_kats(case):
    raw = np.array(case["bytes"], np.uint8)
    got = O.dequantize(case["type"], raw, case["n"])
    for i, e in case["expect"].items():
        assert got[int(i)] == e          # the known answers are exact
    if O.ref() is not None:
        assert np.array_equal(got.view(np.uint32), O.ref_dequantize(case["type"], raw, case["n"]).view(np.uint32))


@pytest.mark.parametrize("case", KATS["dequant_row"], ids=lambda c: f"type{c['type']}_row{c['row']}")
def test_dequant_row_kats(case):
    raw = np.array(case["bytes"], np.uint8)
    out = np.empty(case["cols"], np.float32)
    rc = O.orc().orc_dequantize_row(case["type"], O.ptr(raw), case["nb1"], case["rows"], case["cols"], case["row"],
                                    O.ptr(out))
    assert rc == 0
    assert out.tolist() == case["expect"]
    bad = O.orc().orc_dequantize_row(case["type"], O.ptr(raw), case["nb1"], case["rows"], case["cols"],
                                     case["rows"], O.ptr(out))
    assert bad == -1                     # row out of range (reference src/ds3_reference.c:201-205)
