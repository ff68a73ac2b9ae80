"""The backend as the reference's engine uses it: the reference's own MoE test
built against it, the engine's decode and gathered-prefill call sequences
replayed from C through the ds3_metal_* names, and GGUF-layout weights
imported from a page-aligned mapping with the engine's expert offset table."""
import ctypes as C
import mmap
import subprocess
from pathlib import Path

import numpy as np
import pytest

import _oracle as O
from _cases import Case, assert_close, index_mismatches
from qw3_amd import ds3
from qw3_amd import workload as W
from qw3_amd._native import hip

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
REF_MOE_TEST = ROOT / "oracle" / "_ref" / "test_moe_metal"
HARNESS = ROOT / "tests" / "c" / "_build" / "engine_sequences"
GGUF_ALIGN = 32                   # GGUF tensor data alignment (general.alignment default)


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def test_reference_moe_metal_test(hip_ready):
    """The reference's tests/test_moe_metal.c, unchanged, compiled against
    include/ds3_metal_compat.h and linked with libds3_hip.so: its five
    ds3_metal_moe_ffn cases against its own ds3_reference.c."""
    if not REF_MOE_TEST.exists():
        pytest.skip("oracle/_ref/test_moe_metal was not built (the reference tree was absent at build time)")
    print("  running the reference's test_moe_metal against libds3_hip.so", flush=True)
    r = subprocess.run([str(REF_MOE_TEST)], capture_output=True, text=True, timeout=300)
    print(r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "All MoE tests PASSED" in r.stderr


def _layer_blob(case: Case, perm=None):
    """GGUF-style tensor data of one layer: router (F32), gate, up, down at
    32-byte aligned offsets; with perm, expert e's matrices sit in slot
    perm[e] of each expert tensor.  Returns (bytes, offsets, table [E][3])."""
    h, s = case.host, case.spec
    E = s.n_expert
    parts = [("router", h.router), ("gate", h.gate), ("up", h.up), ("down", h.down)]
    off, offs = 0, {}
    for name, a in parts:
        off = _align(off, GGUF_ALIGN)
        offs[name] = off
        off += a.nbytes
    blob = np.zeros(_align(off, 4096), np.uint8)
    table = np.zeros((E, 3), np.uint64)
    for j, (name, a) in enumerate(parts):
        if name == "router" or perm is None:
            blob[offs[name]:offs[name] + a.nbytes] = a
        else:
            per = a.nbytes // E
            src = a.reshape(E, per)
            for e in range(E):
                blob[offs[name] + perm[e] * per: offs[name] + (perm[e] + 1) * per] = src[e]
        if name != "router":
            per = a.nbytes // E
            table[:, j - 1] = (np.arange(E) if perm is None else np.asarray(perm)) * per
    return blob, offs, table


def test_engine_call_sequences(hip_ready, tmp_path):
    """tests/c/engine_sequences.c replays the engine's decode sequence
    (rms_norm, moe_ffn_router, topk_batch, host read-back, moe_ffn_experts,
    vec_add) and its gathered prefill (per-token router, topk_batch_tokens,
    host bucketing, gather / matmul_quantized_batch x3 / silu_mul /
    scatter_add per expert, vec_add) on a Q4_K/Q6_K layer imported with
    buffer_from_mmap, then the device-routed sequences that replace the
    read-back and host bucketing: the GPU-only decode through moe_ffn with the
    expert offset table (src/ds3_engine.c:638-720), moe_block per token, the
    same block calls as one captured graph, and the prefill chunk through one
    moe_ffn_batch call.  Every sequence matches the oracle on the same
    normalised rows; the device-routed ones match the legacy sequence of
    their kind (indices identical, MoE outputs within the bar), and the
    graph replay equals the eager block calls bit for bit."""
    if not HARNESS.exists():
        pytest.skip("tests/c/_build/engine_sequences was not built")
    spec = W.LayerSpec(n_expert=32)
    case = Case(spec, seed=8080)
    E, K, F, k, T = spec.n_expert, spec.n_embd, spec.n_ff, W.N_USED, 24
    blob, offs, _ = _layer_blob(case)
    hidden = W.fill(W.NORMAL, 81, 1, T * K, 0.0, 1.0).reshape(T, K)
    gain = (1.0 + W.fill(W.NORMAL, 82, 1, K, 0.0, 0.02)).astype(np.float32)
    residual = W.fill(W.NORMAL, 83, 1, T * K, 0.0, 1.0).reshape(T, K)
    blob.tofile(tmp_path / "weights.bin")
    hidden.tofile(tmp_path / "hidden.f32")
    gain.tofile(tmp_path / "gain.f32")
    residual.tofile(tmp_path / "residual.f32")
    (tmp_path / "meta.txt").write_text(
        f"{E} {K} {F} {k} {T} {spec.gate_type} {spec.up_type} {spec.down_type} "
        f"{offs['router']} {offs['gate']} {offs['up']} {offs['down']} {blob.nbytes}\n")
    print(f"  engine call sequences, E={E} T={T}", flush=True)
    r = subprocess.run([str(HARNESS), str(tmp_path)], capture_output=True, text=True, timeout=300)
    print(r.stderr[-1500:], flush=True)
    assert r.returncode == 0, r.stderr[-2000:]
    norm = np.fromfile(tmp_path / "norm.f32", np.float32).reshape(T, K)
    moe, oi, _, probs = case.oracle(norm)
    want = moe + residual
    load = lambda name, dt=np.float32, n=K: np.fromfile(tmp_path / name, dt).reshape(T, n)
    legacy = {}
    for what in ("decode", "prefill"):
        got = load(f"{what}_out.f32")
        gi = load(f"{what}_idx.i32", np.int32, k)
        print(f"    {what}", flush=True)
        assert index_mismatches(gi, oi, probs) == 0
        assert_close(got, want)
        legacy[what] = (got - residual, gi)
    # the device-routed replacements of the read-back and host bucketing, on
    # the same inputs: against the oracle, and their MoE parts and routing
    # against the legacy sequence of the same kind (decode or prefill)
    base = {"gpuonly": residual, "block": hidden, "graph": hidden, "batch": residual}
    kind = {"gpuonly": "decode", "block": "decode", "graph": "decode", "batch": "prefill"}
    for what, x0 in base.items():
        got = load(f"{what}_out.f32")
        print(f"    {what}", flush=True)
        assert_close(got, moe + x0)
        lmoe, lidx = legacy[kind[what]]
        assert_close(got - x0, lmoe.astype(np.float64))
        idx_file = tmp_path / f"{what}_idx.i32"
        if idx_file.exists():
            gi = load(f"{what}_idx.i32", np.int32, k)
            assert index_mismatches(gi, oi, probs) == 0
            assert np.array_equal(gi, lidx)
    # the captured graph replays the eager block calls bit for bit
    assert np.array_equal(load("graph_out.f32").view(np.uint32), load("block_out.f32").view(np.uint32))


def test_gguf_residency_offset_table(hip_ready):
    """A layer in GGUF layout in a page-aligned host mapping, its experts
    stored in shuffled slots: buffer_from_mmap imports it (writes refused,
    views inherit the refusal), the [E][3] offset table is built the way
    upload_expert_offsets builds it (expert slot * rows * nb[1]), and the
    decode and grouped paths read each expert through the table: outputs
    match the oracle on the unshuffled weights."""
    spec = W.config_spec(2)
    case = Case(spec, seed=9090)
    E, K, F, k = spec.n_expert, spec.n_embd, spec.n_ff, W.N_USED
    perm = np.random.default_rng(17).permutation(E)
    blob, offs, table = _layer_blob(case, perm)
    mm = mmap.mmap(-1, blob.nbytes)
    mm.write(blob.tobytes())
    addr = C.addressof(C.c_char.from_buffer(mm))
    assert addr % 4096 == 0
    h = hip().ds3_hip_buffer_from_mmap(addr, blob.nbytes)
    assert h
    wbuf = ds3.Buffer(h, blob.nbytes)
    one = np.zeros(1, np.uint8)
    assert hip().ds3_hip_buffer_write(wbuf, 0, one.ctypes.data, 1) == -1
    h_mis = hip().ds3_hip_buffer_from_mmap(addr + 16, 4096)          # not page-aligned: refused
    assert not h_mis
    gs, us, dsd = (ds3.row_bytes(spec.gate_type, K), ds3.row_bytes(spec.up_type, K),
                   ds3.row_bytes(spec.down_type, F))
    router = wbuf.view(offs["router"], E * K * 4)
    ex = ds3.ExpertTensors(wbuf.view(offs["gate"], E * F * gs), wbuf.view(offs["up"], E * F * us),
                           wbuf.view(offs["down"], E * K * dsd), spec.gate_type, spec.up_type, spec.down_type, K, F)
    assert hip().ds3_hip_buffer_write(ex.gate, 0, one.ctypes.data, 1) == -1
    tbl = ds3.Buffer.from_array(table)
    for T in (1, 64):
        x = W.make_inputs(2, T, seed=900 + T)
        want, oi, _, probs = case.oracle(x)
        out = ds3.Buffer.alloc(T * K * 4)
        idx = ds3.Buffer.alloc(T * k * 4)
        print(f"  residency + offset table, T={T}", flush=True)
        if T == 1:
            logits = ds3.Buffer.alloc(E * 4)
            ds3.moe_ffn(ds3.Buffer.from_array(x), router, spec.router_type, ex, out, logits, E, k,
                        expert_offsets=tbl)
        else:
            ds3.moe_ffn_batch(ds3.Buffer.from_array(x), router, spec.router_type, ex, out, T, E, k, indices=idx,
                              expert_offsets=tbl)
            assert index_mismatches(idx.read(np.int32, (T, k)), oi, probs) == 0
        assert_close(out.read(np.float32, (T, K)), want)
    del ex, router, wbuf
    mm.close()
