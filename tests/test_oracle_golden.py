"""Oracle restatement against vectors written by the compiled reference
(tests/golden/ref_vectors.npz, produced by tests/golden/make_golden.py).
Bit-exact: the restatement performs the same float operations in the same
order, built with the same flags."""
from pathlib import Path

import numpy as np
import pytest

import _oracle as O
from golden.make_golden import MIXED, SMALL, sha, small_inputs
from qw3_amd import ds3

G = np.load(Path(__file__).parent / "golden" / "ref_vectors.npz")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("t,cols", [(ds3.TYPE_Q4_K, 512), (ds3.TYPE_Q6_K, 512), (ds3.TYPE_Q8_0, 128)])
def test_dequant_vectors(t, cols):
    raw = G[f"deq_{t}_raw"]
    got = O.dequantize(t, raw, 4 * cols)
    assert np.array_equal(bits(got), bits(G[f"deq_{t}_out"]))


def test_route_vectors():
    from qw3_amd import workload as W
    lg = W.fill(W.NORMAL, 9, 3, 128 * 16, 0.0, 1.0).reshape(16, 128)
    assert sha(lg) == G["route_logits_sha"].tobytes().hex()
    for i in range(16):
        probs = lg[i].copy()
        O.orc().orc_softmax(O.ptr(probs), 128)
        assert np.array_equal(bits(probs), bits(G["route_probs"][i]))
        idx = np.empty(8, np.int32)
        val = np.empty(8, np.float32)
        O.orc().orc_topk(O.ptr(probs), 128, 8, O.ptr(idx), O.ptr(val))
        assert np.array_equal(idx, G["route_idx"][i])
        assert np.array_equal(bits(val), bits(G["route_val"][i]))


def _orc_moe(x, wr, wg, wu, wd, p):
    E, K, k, Fd = p["n_expert"], p["n_embd"], p["n_used"], p["n_ff"]
    out = np.empty(K, np.float32)
    logits = np.empty(E, np.float32)
    sc = np.empty(k, np.float32)
    idx = np.empty(k, np.int32)
    O.orc().orc_moe_ffn(O.ptr(x), O.ptr(wr), O.ptr(wg), O.ptr(wu), O.ptr(wd), None, None, None, O.ptr(out),
                        O.ptr(logits), O.ptr(sc), O.ptr(idx), K, E, k, Fd, 0, True)
    return out, logits, sc, idx


def test_small_f32_moe_vector():
    x, wr, (wg, wu, wd), _ = small_inputs(SMALL, quant=False)
    assert sha(x, wr, wg, wu, wd) == G["small_inputs_sha"].tobytes().hex()
    out, logits, sc, idx = _orc_moe(x, wr, wg, wu, wd, SMALL)
    assert np.array_equal(idx, G["small_idx"])
    assert np.array_equal(bits(sc), bits(G["small_scores"]))
    assert np.array_equal(bits(logits), bits(G["small_logits"]))
    assert np.array_equal(bits(out), bits(G["small_out"]))


def test_mixed_q4k_q6k_moe_vector():
    x, wr, _, (rg, ru, rd) = small_inputs(MIXED, quant=True)
    assert sha(x, wr, rg, ru, rd) == G["mixed_inputs_sha"].tobytes().hex()
    E, K, Fd = MIXED["n_expert"], MIXED["n_embd"], MIXED["n_ff"]
    dg = O.dequantize(ds3.TYPE_Q4_K, rg, E * Fd * K)
    du = O.dequantize(ds3.TYPE_Q4_K, ru, E * Fd * K)
    dd = O.dequantize(ds3.TYPE_Q6_K, rd, E * K * Fd)
    out, logits, sc, idx = _orc_moe(x, wr, dg, du, dd, MIXED)
    assert np.array_equal(idx, G["mixed_idx"])
    assert np.array_equal(bits(out), bits(G["mixed_out"]))
