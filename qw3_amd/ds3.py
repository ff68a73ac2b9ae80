"""Python host mirror of the ds3_hip C ABI (include/ds3_hip.h).

Thin wrappers that keep the reference's entry-point names and argument
meaning (reference src/ds3_metal.h) and turn a -1 return into an exception.
Device memory is owned by ds3_hip buffers; numpy arrays cross the boundary
through buffer_write / buffer_read.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._native import hip

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 8, 12, 14
TYPE_NAMES = {TYPE_F32: "F32", TYPE_F16: "F16", TYPE_Q8_0: "Q8_0", TYPE_Q4_K: "Q4_K", TYPE_Q6_K: "Q6_K"}
# (values per block, bytes per block) -- reference src/ds3_reference.c:59-184
BLOCK = {TYPE_F32: (1, 4), TYPE_F16: (1, 2), TYPE_Q8_0: (32, 34), TYPE_Q4_K: (256, 144), TYPE_Q6_K: (256, 210)}


class Ds3Error(RuntimeError):
    pass


def row_bytes(type_: int, n_cols: int) -> int:
    per, nb = BLOCK[type_]
    if n_cols % per:
        raise ValueError(f"{n_cols} columns do not fill {TYPE_NAMES[type_]} blocks")
    return n_cols // per * nb


def init() -> None:
    if hip().ds3_hip_init() != 0:
        raise Ds3Error("ds3_hip_init failed (no HIP device?)")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise Ds3Error(f"{what} returned {rc}")


class Buffer:
    """A ds3_hip_buffer_t handle.  Frees its memory when closed or collected.

    Pass the Buffer object itself to ctypes calls (it converts through
    _as_parameter_ and stays referenced for the duration of the call); never
    keep the raw handle of a Buffer that may be collected."""

    def __init__(self, handle: int, nbytes: int, owner: bool = True):
        if not handle:
            raise Ds3Error("buffer allocation failed")
        self.handle = C.c_void_p(handle)
        self.nbytes = nbytes
        self._owner = owner

    @property
    def _as_parameter_(self):
        return self.handle

    @classmethod
    def alloc(cls, nbytes: int) -> "Buffer":
        return cls(hip().ds3_hip_buffer_alloc(nbytes), nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "Buffer":
        a = np.ascontiguousarray(a)
        b = cls.alloc(max(a.nbytes, 1))
        b.write(a)
        return b

    @classmethod
    def from_mmap_array(cls, a: np.ndarray) -> "Buffer":
        """A read-only device copy of a's bytes, imported the way the engine
        imports its mmap'd GGUF weights (ds3_hip_buffer_from_mmap, from a
        page-aligned anonymous mapping): writes to it are refused, and a
        non-F32 router held in it is expanded to FP32 once, not per call."""
        import mmap
        a = np.ascontiguousarray(a)
        n = max(a.nbytes, 1)
        mm = mmap.mmap(-1, n)
        try:
            host = np.frombuffer(mm, dtype=np.uint8, count=n)
            host[:a.nbytes] = a.reshape(-1).view(np.uint8)
            h = hip().ds3_hip_buffer_from_mmap(host.ctypes.data, n)
            del host
        finally:
            mm.close()
        return cls(h, n)

    def view(self, offset: int, nbytes: int) -> "Buffer":
        return Buffer(hip().ds3_hip_buffer_view(self.handle, offset, nbytes), nbytes, owner=True)

    def write(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        _check(hip().ds3_hip_buffer_write(self.handle, offset, a.ctypes.data, a.nbytes), "buffer_write")

    def read(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _check(hip().ds3_hip_buffer_read(self.handle, offset, out.ctypes.data, out.nbytes), "buffer_read")
        return out

    def zero(self) -> None:
        _check(hip().ds3_hip_buffer_zero_f32(self.handle, self.nbytes - self.nbytes % 4), "buffer_zero_f32")

    def close(self) -> None:
        if self._owner and self.handle:
            hip().ds3_hip_buffer_free(self.handle)
        self.handle = C.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _h(b):
    return b if b is not None else None


@dataclass
class ExpertTensors:
    """Packed expert weights of one layer, expert-major like the GGUF tensors
    ffn_{gate,up,down}_exps (reference src/ds3_engine.c:977-1003)."""
    gate: Buffer
    up: Buffer
    down: Buffer
    gate_type: int
    up_type: int
    down_type: int
    n_embd: int
    n_ff: int

    @property
    def strides(self):
        return (row_bytes(self.gate_type, self.n_embd), row_bytes(self.up_type, self.n_embd),
                row_bytes(self.down_type, self.n_ff))


def dequantize(src: Buffer, type_: int, n: int, dst: Buffer, src_offset: int = 0) -> None:
    _check(hip().ds3_hip_dequantize(src, src_offset, type_, n, dst), "dequantize")


def moe_route(x: Buffer, router: Buffer, router_type: int, n_tokens: int, n_embd: int, n_expert: int,
              n_used: int, indices: Buffer, scores: Buffer, logits: Buffer | None = None,
              norm: bool = True) -> None:
    _check(hip().ds3_hip_moe_route(x, router, _h(logits), indices, scores,
                                   n_tokens, n_embd, n_expert, n_used, row_bytes(router_type, n_embd),
                                   router_type, norm), "moe_route")


def moe_bucket(indices: Buffer, scores: Buffer, n_tokens: int, n_used: int, n_expert: int,
               counts: Buffer, offsets: Buffer, ids: Buffer, wts: Buffer, slot_pos: Buffer) -> None:
    _check(hip().ds3_hip_moe_bucket(indices, scores, n_tokens, n_used, n_expert, counts,
                                    offsets, ids, wts, slot_pos), "moe_bucket")


def moe_ffn_batch(x: Buffer, router: Buffer, router_type: int, ex: ExpertTensors, out: Buffer, n_tokens: int,
                  n_expert: int, n_used: int, residual: Buffer | None = None, logits: Buffer | None = None,
                  indices: Buffer | None = None, scores: Buffer | None = None, norm: bool = True,
                  expert_offsets: Buffer | None = None, noalloc: bool = False) -> None:
    """T tokens through the layer on the device (ds3_hip_moe_ffn_batch; with
    noalloc, ds3_hip_moe_ffn_batch_noalloc: no allocation, intermediates in
    the library's scratch array)."""
    gs, us, ds = ex.strides
    fn = hip().ds3_hip_moe_ffn_batch_noalloc if noalloc else hip().ds3_hip_moe_ffn_batch
    _check(fn(
        x, router, ex.gate, ex.up, ex.down,
        ex.gate_type, ex.up_type, ex.down_type, gs, us, ds, _h(expert_offsets),
        out, _h(residual), _h(logits), _h(indices), _h(scores),
        n_tokens, ex.n_embd, n_expert, n_used, ex.n_ff, row_bytes(router_type, ex.n_embd), router_type, norm),
        "moe_ffn_batch_noalloc" if noalloc else "moe_ffn_batch")


def moe_block(hidden: Buffer, ffn_norm: Buffer, eps: float, router: Buffer, router_type: int, ex: ExpertTensors,
              n_tokens: int, n_expert: int, n_used: int, x_norm: Buffer | None = None, logits: Buffer | None = None,
              indices: Buffer | None = None, scores: Buffer | None = None, norm: bool = True,
              expert_offsets: Buffer | None = None) -> None:
    """The engine's FFN block in place: hidden += MoE(rms_norm(hidden) * ffn_norm)."""
    gs, us, ds = ex.strides
    _check(hip().ds3_hip_moe_block(
        hidden, ffn_norm, eps, router, ex.gate, ex.up, ex.down,
        ex.gate_type, ex.up_type, ex.down_type, gs, us, ds, _h(expert_offsets),
        _h(x_norm), _h(logits), _h(indices), _h(scores),
        n_tokens, ex.n_embd, n_expert, n_used, ex.n_ff, row_bytes(router_type, ex.n_embd), router_type, norm),
        "moe_block")


def rms_norm(x: Buffer, weight: Buffer, out: Buffer, n: int, n_rows: int, eps: float) -> None:
    """ds3_metal_rms_norm-compatible (reference src/ds3_metal.h:48-57)."""
    _check(hip().ds3_hip_rms_norm(x, weight, out, n, n_rows, eps), "rms_norm")


def moe_ffn(x: Buffer, router: Buffer, router_type: int, ex: ExpertTensors, out: Buffer, logits: Buffer,
            n_expert: int, n_used: int, norm: bool = True, scratch: Buffer | None = None,
            shared: ExpertTensors | None = None, n_ff_shared: int = 0, expert_offsets: Buffer | None = None) -> None:
    """ds3_metal_moe_ffn-compatible single-token call (reference src/ds3_metal.h:340-374)."""
    gs, us, ds = ex.strides
    scratch = scratch or Buffer.alloc(4 * max(ex.n_ff, ex.n_embd, n_ff_shared, 1))
    if shared is not None:
        sg, su, sd = shared.gate, shared.up, shared.down
        sgt, sut, sdt = shared.gate_type, shared.up_type, shared.down_type
        sgs, sus = row_bytes(sgt, ex.n_embd), row_bytes(sut, ex.n_embd)
        sds = row_bytes(sdt, n_ff_shared)
    else:
        sg = su = sd = None
        sgt = sut = sdt = TYPE_F32
        sgs = sus = sds = 0
    _check(hip().ds3_hip_moe_ffn(
        x, router, ex.gate, ex.up, ex.down,
        ex.gate_type, ex.up_type, ex.down_type, gs, us, ds,
        sg, su, sd, sgt, sut, sdt, sgs, sus, sds,
        out, logits, _h(expert_offsets), scratch, scratch, scratch,
        ex.n_embd, n_expert, n_used, ex.n_ff, n_ff_shared, row_bytes(router_type, ex.n_embd), router_type, norm),
        "moe_ffn")


class Graph:
    """Calls made inside `with ds3.Graph() as gr:` are captured, not run;
    gr.launch() replays them (ds3_hip_graph_begin / _end / _launch)."""

    def __init__(self):
        self.handle = None

    def __enter__(self) -> "Graph":
        _check(hip().ds3_hip_graph_begin(), "graph_begin")
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        h = C.c_void_p()
        rc = hip().ds3_hip_graph_end(C.byref(h))
        if exc_type is None:
            _check(rc, "graph_end")
            self.handle = h.value
        elif rc == 0 and h.value:
            hip().ds3_hip_graph_destroy(h.value)

    def launch(self) -> None:
        _check(hip().ds3_hip_graph_launch(self.handle), "graph_launch")

    def close(self) -> None:
        if self.handle:
            hip().ds3_hip_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def set_prefill_min_tokens(n: int) -> int:
    return hip().ds3_hip_set_prefill_min_tokens(n)


ROUTER_AUTO, ROUTER_SEQUENTIAL, ROUTER_CERTIFIED = 0, 1, 2


def set_router_mode(mode: int) -> int:
    """Router selection (ds3_hip_set_router_mode); returns the previous mode."""
    return hip().ds3_hip_set_router_mode(mode)


def router_stats(reset: bool = False) -> tuple[int, int]:
    """(tokens certified, tokens repaired) by the certified router."""
    c, r = C.c_uint64(), C.c_uint64()
    _check(hip().ds3_hip_router_stats(C.byref(c), C.byref(r), 1 if reset else 0), "router_stats")
    return c.value, r.value


def grouped_lists() -> dict:
    """The bucketing lists of the last chunk of the last grouped-path call
    (ds3_hip_debug_grouped_lists) and its run descriptors
    (ds3_hip_debug_grouped_descs), as numpy arrays."""
    h = hip()
    meta = np.zeros(12, np.int32)
    _check(h.ds3_hip_debug_grouped_lists(meta.ctypes.data, *([None] * 8)), "debug_grouped_lists")
    t0, tc, k, E, nt, ngu, ndn, marked, rpi_gu, rpi_dn, max_tiles, tile_m = (int(v) for v in meta)
    S = tc * k
    a = {"counts": np.zeros(E, np.int32), "offsets": np.zeros(E + 1, np.int32), "ids": np.zeros(S, np.int32),
         "wts": np.zeros(S, np.float32), "slot_pos": np.zeros(S, np.int32), "tiles": np.zeros(nt, np.int32),
         "runs_gu": np.zeros(ngu, np.int32), "runs_dn": np.zeros(ndn, np.int32)}
    _check(h.ds3_hip_debug_grouped_lists(meta.ctypes.data, *(v.ctypes.data for v in a.values())),
           "debug_grouped_lists")
    dg, dd = np.zeros((ngu, 2), np.int32), np.zeros((ndn, 2), np.int32)
    _check(h.ds3_hip_debug_grouped_descs(dg.ctypes.data, dd.ctypes.data), "debug_grouped_descs")
    a.update(desc_gu=dg, desc_dn=dd)
    a.update(t0=t0, tc=tc, k=k, E=E, marked=bool(marked), rpi_gu=rpi_gu, rpi_dn=rpi_dn, max_tiles=max_tiles,
             tile_m=tile_m)
    return a


def device_info() -> dict:
    arch = C.create_string_buffer(64)
    ncu = C.c_int()
    hbm = C.c_uint64()
    _check(hip().ds3_hip_device_info(arch, 64, C.byref(ncu), C.byref(hbm)), "device_info")
    return {"arch": arch.value.decode(), "n_cu": ncu.value, "hbm_bytes": hbm.value}


def kernel_stats() -> dict[str, tuple[int, float]]:
    """{kernel: (launches, total_ms)} recorded while kernel timing was on."""
    out = {}
    name = C.create_string_buffer(128)
    cnt, ms = C.c_int64(), C.c_double()
    i = 0
    while hip().ds3_hip_kernel_stats(i, name, 128, C.byref(cnt), C.byref(ms)) == 0:
        out[name.value.decode()] = (cnt.value, ms.value)
        i += 1
    return out
