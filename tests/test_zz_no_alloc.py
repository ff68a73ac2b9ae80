"""The allocation-free entry point ds3_hip_moe_ffn_batch_noalloc against
ds3_hip_moe_ffn_batch, through the C ABI: identical outputs, indices, scores
and logits on consecutive calls (the second smaller, so it runs on what the
first left in the shared scratch array), a clear refusal of a call whose
intermediates exceed the scratch array, and the documented capacity edge."""
import numpy as np
import pytest

from _cases import Case
from qw3_amd import ds3
from qw3_amd import workload as W
from qw3_amd._native import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer():
    print("  building config-2 layer", flush=True)
    return Case(W.config_spec(2), seed=5050)


def _run(case, x, T, noalloc, residual=None):
    s = case.spec
    out = ds3.Buffer.from_array(np.full((T, s.n_embd), 0.25, np.float32))     # accumulates into this
    idx, sc = ds3.Buffer.alloc(T * W.N_USED * 4), ds3.Buffer.alloc(T * W.N_USED * 4)
    lg = ds3.Buffer.alloc(T * s.n_expert * 4)
    ds3.moe_ffn_batch(x, case.dev.router, s.router_type, case.dev.experts, out, T, s.n_expert, W.N_USED,
                      residual=residual, logits=lg, indices=idx, scores=sc, noalloc=noalloc)
    return (out.read(np.float32, (T, s.n_embd)), idx.read(np.int32, (T, W.N_USED)),
            sc.read(np.float32, (T, W.N_USED)), lg.read(np.float32, (T, s.n_expert)))


def test_noalloc_matches_allocating_entry_point(hip_ready, layer):
    assert hip().ds3_hip_noalloc_scratch_bytes() == 64 << 20
    s = layer.spec
    # grouped path, then a smaller grouped call, then decode paths (fused
    # selection at T = 1, separate selection at T = 4)
    for T in (512, 64, 1, 4):
        print(f"  noalloc vs allocating, T={T}", flush=True)
        x = ds3.Buffer.from_array(W.make_inputs(2, T, seed=600 + T))
        res = ds3.Buffer.from_array(W.make_inputs(2, T, seed=700 + T)) if T == 64 else None
        want = _run(layer, x, T, False, res)
        got = _run(layer, x, T, True, res)
        for g, w, what in zip(got, want, ("output", "indices", "scores", "logits")):
            assert np.array_equal(g, w), f"T={T}: {what} differ"


def test_noalloc_refuses_oversized_call(hip_ready, layer, capfd):
    s = layer.spec
    T = 4096                                       # y alone needs 64 MiB per 2048-token chunk, h 24 MiB
    x = ds3.Buffer.alloc(T * s.n_embd * 4)
    out = ds3.Buffer.alloc(T * s.n_embd * 4)
    ex = layer.dev.experts
    gs, us, dsd = ex.strides
    rc = hip().ds3_hip_moe_ffn_batch_noalloc(
        x, layer.dev.router, ex.gate, ex.up, ex.down, ex.gate_type, ex.up_type, ex.down_type, gs, us, dsd, None,
        out, None, None, None, None, T, s.n_embd, s.n_expert, W.N_USED, s.n_ff,
        ds3.row_bytes(s.router_type, s.n_embd), s.router_type, True)
    assert rc == -1
    assert "allocation-free entry point holds" in capfd.readouterr().err
    # the entry point still works after the refusal
    xs = ds3.Buffer.from_array(W.make_inputs(2, 16, seed=800))
    got, want = _run(layer, xs, 16, True), _run(layer, xs, 16, False)
    assert all(np.array_equal(g, w) for g, w in zip(got, want))


def test_noalloc_capacity_edge(hip_ready, layer):
    """The documented capacity for a Qwen3-30B-A3B layer call: 1,284 tokens
    fit the scratch array (and match the allocating entry point), 1,285 are
    refused."""
    s = layer.spec
    T = 1284
    print(f"  noalloc at its capacity, T={T}", flush=True)
    x = ds3.Buffer.from_array(W.make_inputs(2, T, seed=900))
    got, want = _run(layer, x, T, True), _run(layer, x, T, False)
    assert all(np.array_equal(g, w) for g, w in zip(got, want))
    T = 1285
    print(f"  noalloc one token past it, T={T}", flush=True)
    x = ds3.Buffer.alloc(T * s.n_embd * 4)
    out = ds3.Buffer.alloc(T * s.n_embd * 4)
    ex = layer.dev.experts
    gs, us, dsd = ex.strides
    rc = hip().ds3_hip_moe_ffn_batch_noalloc(
        x, layer.dev.router, ex.gate, ex.up, ex.down, ex.gate_type, ex.up_type, ex.down_type, gs, us, dsd, None,
        out, None, None, None, None, T, s.n_embd, s.n_expert, W.N_USED, s.n_ff,
        ds3.row_bytes(s.router_type, s.n_embd), s.router_type, True)
    assert rc == -1
