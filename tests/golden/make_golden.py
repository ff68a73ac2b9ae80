"""Write the golden fixtures of tests/golden/.

1. reference_kats.json -- the known-answer inputs and expected values held in
   the reference's unit tests (tests/test_reference.c:32-468), restated as data.
2. ref_vectors.npz -- outputs of the reference's own ds3_reference.c, compiled
   from its sources into oracle/_ref/libds3ref.so (oracle/Makefile), on inputs
   from this project's deterministic generator.  Inputs are regenerated at test
   time from (seed, stream); the fixture stores their SHA-256 so a generator
   change is caught, plus raw quantised bytes where they are small.

Run from the repository root after `make -C oracle` and building qw3_amd:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import _oracle as O  # noqa: E402
from qw3_amd import workload as W  # noqa: E402
from qw3_amd import ds3  # noqa: E402


def kats() -> dict:
    """Known answers of the reference's tests/test_reference.c, as data."""
    q4k = np.zeros(144, np.uint8)
    q4k[0:2] = [0x00, 0x3C]          # d = 1.0
    q4k[2:4] = [0x00, 0x3C]          # dmin = 1.0
    sc = q4k[4:16]
    sc[0], sc[1], sc[4], sc[5], sc[8], sc[9] = 1, 1, 0, 0, 0x53, 0x02
    q4k[16 + 0] = 0xAB
    q4k[16 + 64] = 0xCD
    q80 = np.zeros(34, np.uint8)
    q80[0:2] = [0x00, 0x3C]
    q80[2] = 5
    q80[3] = 0xFD                    # -3
    q6k = np.zeros(210, np.uint8)
    q6k[208:210] = [0x00, 0x3C]
    q6k[192:208] = 1
    q6k[0] = 0x31
    q6k[32] = 0x42
    q6k[128] = 0xAA
    rms = float(np.sqrt(np.float32(7.5)))
    return {
        "source": "reference tests/test_reference.c (EPS 1e-4, line 15)",
        "eps": 1e-4,
        "rms_norm": {"x": [1, 2, 3, 4], "cases": [
            {"w": [1, 1, 1, 1], "eps": 1e-6, "expect": {"0": 1 / rms, "1": 2 / rms, "2": 3 / rms, "3": 4 / rms}},
            {"w": [2, 2, 2, 2], "eps": 1e-6, "expect": {"0": 2 / rms, "3": 8 / rms}}]},
        "softmax": [
            {"x": [1, 2, 3, 4], "expect": {"0": 0.0320586, "3": 0.6439143}, "sum": 1.0},
            {"x": [5, 5, 5, 5], "expect": {"0": 0.25}, "sum": 1.0}],
        "silu": {"x": [0.0, 1.0, -1.0],
                 "expect": [0.0, float(1 / (1 + np.exp(np.float32(-1)))), float(-1 / (1 + np.exp(np.float32(1))))]},
        "topk": {"scores": [0.1, 0.5, 0.2, 0.9, 0.3, 0.8, 0.0, 0.4], "k": 3,
                 "idx": [3, 5, 1], "val": [0.9, 0.8, 0.5]},
        "dequant": [
            {"type": ds3.TYPE_Q4_K, "n": 256, "bytes": q4k.tolist(),
             "expect": {"0": 11, "32": 10, "1": 0, "33": 0, "128": 34, "160": 24, "129": -5, "161": 0}},
            {"type": ds3.TYPE_Q8_0, "n": 32, "bytes": q80.tolist(), "expect": {"0": 5, "1": -3, "2": 0}},
            {"type": ds3.TYPE_Q6_K, "n": 256, "bytes": q6k.tolist(), "expect": {"0": 1, "32": 2, "64": 3, "96": 4}},
            {"type": ds3.TYPE_F16, "n": 3, "bytes": [0x00, 0x3C, 0x00, 0x40, 0x00, 0x00],
             "expect": {"0": 1, "1": 2, "2": 0}}],
        "dequant_row": [
            {"type": ds3.TYPE_F32, "rows": 2, "cols": 3, "nb1": 12,
             "bytes": np.arange(1, 7, dtype=np.float32).view(np.uint8).tolist(), "row": 1, "expect": [4, 5, 6]},
            {"type": ds3.TYPE_F16, "rows": 2, "cols": 3, "nb1": 6,
             "bytes": np.array([0x3C00, 0x4000, 0x0000, 0x4200, 0x4400, 0x4500], np.uint16).view(np.uint8).tolist(),
             "row": 0, "expect": [1, 2, 0]},
            {"type": ds3.TYPE_F16, "rows": 2, "cols": 3, "nb1": 6,
             "bytes": np.array([0x3C00, 0x4000, 0x0000, 0x4200, 0x4400, 0x4500], np.uint16).view(np.uint8).tolist(),
             "row": 1, "expect": [3, 4, 5]}],
    }


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


SMALL = dict(n_embd=256, n_expert=16, n_used=4, n_ff=128, seed=70)
MIXED = dict(n_embd=512, n_expert=16, n_used=4, n_ff=256, seed=72)


def small_inputs(p: dict, quant: bool):
    E, K, Fd = p["n_expert"], p["n_embd"], p["n_ff"]
    s = p["seed"]
    x = W.fill(W.NORMAL, s, W.stream_id(0, W.K_X), K, 0.0, 1.0)
    wr = W.fill(W.NORMAL, s, W.stream_id(0, W.K_ROUTER), E * K, 0.0, 0.1).reshape(E, K)
    if not quant:
        wg = W.fill(W.NORMAL, s, W.stream_id(0, W.K_GATE), E * Fd * K, 0.0, 0.05)
        wu = W.fill(W.NORMAL, s, W.stream_id(0, W.K_UP), E * Fd * K, 0.0, 0.05)
        wd = W.fill(W.NORMAL, s, W.stream_id(0, W.K_DOWN), E * K * Fd, 0.0, 0.05)
        return x, wr, (wg, wu, wd), None
    rg = W.quant_matrix(ds3.TYPE_Q4_K, W.NORMAL, s, W.stream_id(0, W.K_GATE), E * Fd, K, 0.0, 0.05)
    ru = W.quant_matrix(ds3.TYPE_Q4_K, W.NORMAL, s, W.stream_id(0, W.K_UP), E * Fd, K, 0.0, 0.05)
    rd = W.quant_matrix(ds3.TYPE_Q6_K, W.NORMAL, s, W.stream_id(0, W.K_DOWN), E * K, Fd, 0.0, 0.05)
    return x, wr, None, (rg, ru, rd)


def ref_moe(x, wr, wg, wu, wd, p):
    r = O.ref()
    E, K, k, Fd = p["n_expert"], p["n_embd"], p["n_used"], p["n_ff"]
    out = np.empty(K, np.float32)
    logits = np.empty(E, np.float32)
    sc = np.empty(k, np.float32)
    idx = np.empty(k, np.int32)
    r.ds3_ref_moe_ffn(O.ptr(x), O.ptr(wr), O.ptr(wg), O.ptr(wu), O.ptr(wd), None, None, None, O.ptr(out),
                      O.ptr(logits), O.ptr(sc), O.ptr(idx), K, E, k, Fd, 0, True)
    return out, logits, sc, idx


def vectors() -> dict:
    assert O.ref() is not None, "oracle/_ref/libds3ref.so missing: run make -C oracle"
    out = {}
    # dequantisation of generator-quantised blocks
    for t, cols in ((ds3.TYPE_Q4_K, 512), (ds3.TYPE_Q6_K, 512), (ds3.TYPE_Q8_0, 128)):
        raw = W.quant_matrix(t, W.NORMAL, 5, 77 + t, 4, cols, 0.0, 0.02)
        out[f"deq_{t}_raw"] = raw
        out[f"deq_{t}_out"] = O.ref_dequantize(t, raw, 4 * cols)
    # softmax / top-k / renorm on seeded logits
    lg = W.fill(W.NORMAL, 9, 3, 128 * 16, 0.0, 1.0).reshape(16, 128)
    probs = lg.copy()
    idx = np.empty((16, 8), np.int32)
    val = np.empty((16, 8), np.float32)
    for i in range(16):
        O.ref().ds3_ref_softmax(O.ptr(probs[i]), 128)
        O.ref().ds3_ref_topk(O.ptr(probs[i]), 128, 8, O.ptr(idx[i]), O.ptr(val[i]))
    out["route_logits_sha"] = np.frombuffer(bytes.fromhex(sha(lg)), np.uint8)
    out["route_probs"], out["route_idx"], out["route_val"] = probs, idx, val
    # small F32 MoE (shape of reference tests/test_moe_metal.c:26-118)
    x, wr, (wg, wu, wd), _ = small_inputs(SMALL, quant=False)
    o, l, s, i = ref_moe(x, wr, wg, wu, wd, SMALL)
    out["small_inputs_sha"] = np.frombuffer(bytes.fromhex(sha(x, wr, wg, wu, wd)), np.uint8)
    out["small_out"], out["small_logits"], out["small_scores"], out["small_idx"] = o, l, s, i
    # mixed Q4_K gate/up + Q6_K down MoE (shape of test_moe_metal.c:509-659, reduced)
    x, wr, _, (rg, ru, rd) = small_inputs(MIXED, quant=True)
    E, K, Fd = MIXED["n_expert"], MIXED["n_embd"], MIXED["n_ff"]
    dg = O.ref_dequantize(ds3.TYPE_Q4_K, rg, E * Fd * K)
    du = O.ref_dequantize(ds3.TYPE_Q4_K, ru, E * Fd * K)
    dd = O.ref_dequantize(ds3.TYPE_Q6_K, rd, E * K * Fd)
    o, l, s, i = ref_moe(x, wr, dg, du, dd, MIXED)
    out["mixed_inputs_sha"] = np.frombuffer(bytes.fromhex(sha(x, wr, rg, ru, rd)), np.uint8)
    out["mixed_out"], out["mixed_logits"], out["mixed_scores"], out["mixed_idx"] = o, l, s, i
    return out


if __name__ == "__main__":
    (HERE / "reference_kats.json").write_text(json.dumps(kats(), indent=1) + "\n")
    np.savez_compressed(HERE / "ref_vectors.npz", **vectors())
    print("wrote", HERE / "reference_kats.json", HERE / "ref_vectors.npz")
