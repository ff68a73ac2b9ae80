"""Configuration 4 at full size: one token per step through 48 resident
Qwen3-30B-A3B MoE layers (17.5 GiB of Q4_K/Q6_K experts), as the engine runs
decode (reference src/ds3_engine.c:515-588: the FFN block once per layer,
h += MoE(rms_norm(h) * g)).  The captured graph of the whole stack must
reproduce the eager calls bit for bit, and the first, middle and last
layers are checked against the oracle on the device's own input to them
(teacher forcing)."""
import numpy as np
import pytest

from _cases import Case, assert_close, index_mismatches
from qw3_amd import ds3
from qw3_amd import workload as W
from qw3_amd._native import hip

pytestmark = pytest.mark.gpu

N_LAYERS = 48
CHECKED = (0, 23, 47)


@pytest.fixture(scope="module")
def stack():
    spec = W.config_spec(4)
    K = spec.n_embd
    print(f"  generating {N_LAYERS} resident layers", flush=True)
    layers, hosts = [], {}
    for l in range(N_LAYERS):
        h = W.make_layer(spec, seed=1234, layer=l)
        layers.append(h.to_device())
        if l in CHECKED:
            hosts[l] = h
    gains = [ds3.Buffer.from_array((1.0 + W.fill(W.NORMAL, 700 + l, 1, K, 0.0, 0.02)).astype(np.float32))
             for l in range(N_LAYERS)]
    yield spec, layers, hosts, gains
    del layers, gains
    hip().ds3_hip_synchronize()


def _layer(spec, d, h, gain, ix=None):
    if gain is None:
        ds3.moe_ffn_batch(h, d.router, spec.router_type, d.experts, h, 1, spec.n_expert, W.N_USED, indices=ix)
    else:
        ds3.moe_block(h, gain, 1e-6, d.router, spec.router_type, d.experts, 1, spec.n_expert, W.N_USED,
                      indices=ix)


@pytest.mark.parametrize("block", [False, True], ids=["ffn", "block"])
def test_stack_graph_equals_eager(hip_ready, stack, block):
    """Eager tokens through the 48 layers, then the same tokens through one
    captured graph of the 48 layer calls: identical bits, every replay."""
    spec, layers, _, gains = stack
    K = spec.n_embd
    h = ds3.Buffer.alloc(K * 4)
    xs = [W.make_inputs(4, 1, seed=99, step=s) for s in range(3)]
    eager = []
    for i, x in enumerate(xs):
        print(f"  eager token {i} ({'block' if block else 'ffn'})", flush=True)
        h.write(x)
        for l, d in enumerate(layers):
            _layer(spec, d, h, gains[l] if block else None)
        eager.append(h.read(np.float32, (1, K)))
    assert all(np.isfinite(e).all() for e in eager)
    with ds3.Graph() as gr:
        for l, d in enumerate(layers):
            _layer(spec, d, h, gains[l] if block else None)
    try:
        for rep in range(2):
            for i, x in enumerate(xs):
                h.write(x)
                gr.launch()
                got = h.read(np.float32, (1, K))
                assert np.array_equal(got, eager[i]), f"replay {rep} token {i}"
    finally:
        gr.close()


def test_stack_teacher_forced_deep_layers(hip_ready, stack):
    """One token through all 48 layers eagerly, the hidden state read after
    every layer; layers 0, 23 and 47 recomputed by the oracle from the
    device's input to them: experts selected alike (or tied) and
    h_out = h_in + MoE(h_in) within the output tolerance."""
    spec, layers, hosts, _ = stack
    K = spec.n_embd
    h = ds3.Buffer.alloc(K * 4)
    idx = ds3.Buffer.alloc(W.N_USED * 4)
    h.write(W.make_inputs(4, 1, seed=99, step=5))
    states = [h.read(np.float32, (1, K))]
    picked = {}
    for l, d in enumerate(layers):
        _layer(spec, d, h, None, idx if l in CHECKED else None)
        states.append(h.read(np.float32, (1, K)))
        if l in CHECKED:
            picked[l] = idx.read(np.int32, (1, W.N_USED))
    print(f"  |h| after 48 layers: {float(np.linalg.norm(states[-1])):.3f}", flush=True)
    for l in CHECKED:
        case = Case(spec, host=hosts[l])            # dequantises the layer's host copy
        h_in = states[l]
        want, oi, _, probs = case.oracle(h_in)
        print(f"  layer {l}", flush=True)
        assert index_mismatches(picked[l], oi, probs) == 0
        assert_close(states[l + 1], h_in + want, max_abs=3e-3, rel_l2=1.2e-3)
        del case
