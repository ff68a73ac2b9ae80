"""Host-runtime safety on the GPU: captured graphs keep the workspace block
their kernels address when an eager call grows the workspace, and entry points
that would break an open capture refuse instead."""
import numpy as np
import pytest

from _cases import Case
from qw3_amd import ds3
from qw3_amd import workload as W
from qw3_amd._native import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer():
    print("  building Q4_K/Q6_K layer", flush=True)
    return Case(W.config_spec(2), seed=4040)


def _call(case, x, out, T, idx=None):
    s = case.spec
    out.zero()                                       # a fill kernel, not a memset node
    ds3.moe_ffn_batch(x, case.dev.router, s.router_type, case.dev.experts, out, T, s.n_expert, W.N_USED,
                      indices=idx)


def _fresh_context():
    """Shut the context down and initialise it again: the workspace starts
    empty, so the next large call is sure to grow it."""
    hip().ds3_hip_shutdown()
    ds3.init()


def test_graph_survives_workspace_growth(hip_ready, layer):
    """Capture a T=1 call, grow the workspace with an eager T=512 call (the
    captured kernels' block is retired, not freed), replay: bit-equal to the
    eager T=1 result, every replay; then destroying the graph frees the
    retired block and eager calls still match."""
    s = layer.spec
    _fresh_context()
    x1 = ds3.Buffer.from_array(W.make_inputs(2, 1, seed=301))
    x512 = ds3.Buffer.from_array(W.make_inputs(2, 512, seed=302))
    o1, i1 = ds3.Buffer.alloc(s.n_embd * 4), ds3.Buffer.alloc(W.N_USED * 4)
    o512 = ds3.Buffer.alloc(512 * s.n_embd * 4)
    print("  eager T=1, capture T=1", flush=True)
    _call(layer, x1, o1, 1, i1)
    want1, want_i = o1.read(np.float32, (1, s.n_embd)), i1.read(np.int32, (1, W.N_USED))
    with ds3.Graph() as gr:
        _call(layer, x1, o1, 1, i1)
    try:
        print("  eager T=512 (grows the workspace), then replays", flush=True)
        _call(layer, x512, o512, 512)
        want512 = o512.read(np.float32, (512, s.n_embd))
        for rep in range(3):
            o1.write(np.full((1, s.n_embd), 5.0, np.float32))
            i1.write(np.full((1, W.N_USED), -1, np.int32))
            gr.launch()
            assert np.array_equal(o1.read(np.float32, (1, s.n_embd)), want1), f"replay {rep}"
            assert np.array_equal(i1.read(np.int32, (1, W.N_USED)), want_i), f"replay {rep}"
            _call(layer, x512, o512, 512)              # eager work on the new block between replays
            assert np.array_equal(o512.read(np.float32, (512, s.n_embd)), want512)
    finally:
        gr.close()
    _call(layer, x1, o1, 1)
    assert np.array_equal(o1.read(np.float32, (1, s.n_embd)), want1)


def test_graph_after_shutdown_is_refused(hip_ready, layer):
    """ds3_hip_shutdown destroys live graphs: a later launch of one returns -1."""
    s = layer.spec
    x1 = ds3.Buffer.from_array(W.make_inputs(2, 1, seed=303))
    o1 = ds3.Buffer.alloc(s.n_embd * 4)
    _call(layer, x1, o1, 1)
    with ds3.Graph() as gr:
        _call(layer, x1, o1, 1)
    _fresh_context()
    assert hip().ds3_hip_graph_launch(gr.handle) == -1
    gr.close()                                      # destroying a graph the shutdown ended is a no-op
    _call(layer, x1, o1, 1)


def test_capture_refusals(hip_ready, layer):
    """Inside a real capture: allocation, host copies, host-index expert calls
    and waits refuse; a freed buffer is released at graph_end; the capture
    itself stays valid and its replay equals the eager call."""
    s = layer.spec
    T = 4
    x = ds3.Buffer.from_array(W.make_inputs(2, T, seed=304))
    out = ds3.Buffer.alloc(T * s.n_embd * 4)
    spare = ds3.Buffer.alloc(4096)
    _call(layer, x, out, T)
    want = out.read(np.float32, (T, s.n_embd))
    ex = layer.dev.experts
    gs, us, dsd = ex.strides
    idx = (np.arange(W.N_USED, dtype=np.int32))
    sc = np.full(W.N_USED, 1.0 / W.N_USED, np.float32)
    with ds3.Graph() as gr:
        _call(layer, x, out, T)
        with pytest.raises(ds3.Ds3Error):
            ds3.Buffer.alloc(4096)
        with pytest.raises(ds3.Ds3Error):
            spare.read(np.uint8, (16,))
        with pytest.raises(ds3.Ds3Error):
            spare.write(np.zeros(16, np.uint8))
        rc = hip().ds3_hip_moe_ffn_experts(
            x, ex.gate, ex.up, ex.down, ex.gate_type, ex.up_type, ex.down_type, gs, us, dsd,
            None, None, None, 0, 0, 0, 0, 0, 0, out, None, spare, spare, s.n_embd, W.N_USED, s.n_ff, 0,
            idx.ctypes.data_as(ds3.C.POINTER(ds3.C.c_int32)), sc.ctypes.data_as(ds3.C.POINTER(ds3.C.c_float)))
        assert rc == -1
        hip().ds3_hip_synchronize()                  # refused: a no-op inside the capture
        spare.close()                                # deferred to graph_end
    try:
        for rep in range(2):
            out.write(np.full((T, s.n_embd), 3.0, np.float32))
            gr.launch()
            assert np.array_equal(out.read(np.float32, (T, s.n_embd)), want), f"replay {rep}"
    finally:
        gr.close()
