"""ctypes bindings of the CPU oracle (oracle/liboracle.so) and, where it was
built, the reference's own ds3_reference.c (oracle/_ref/libds3ref.so).

Test infrastructure only.  Helpers here run the oracle on the same seeded
inputs the GPU receives.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libds3ref.so"

P, I, F, B = C.c_void_p, C.c_int, C.c_float, C.c_bool
I64, SZ, U64 = C.c_int64, C.c_size_t, C.c_uint64

_ORC = {
    "orc_fp16_to_fp32": (F, [C.c_uint16]),
    "orc_row_bytes": (SZ, [I, I64]),
    "orc_dequantize": (I, [I, P, SZ, I64, P]),
    "orc_dequantize_row": (I, [I, P, U64, I64, I64, I, P]),
    "orc_vec_matmul": (None, [P, P, P, I, I]),
    "orc_softmax": (None, [P, I]),
    "orc_topk": (I, [P, I, I, P, P]),
    "orc_silu": (None, [P, P, I]),
    "orc_mul": (None, [P, P, P, I]),
    "orc_add": (None, [P, P, P, I]),
    "orc_rms_norm": (None, [P, P, F, I, P]),
    "orc_route": (None, [P, I, I, B, P, P]),
    "orc_moe_ffn": (None, [P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, B]),
    "orc_moe_ffn_tokens": (I, [I, P, P, P, P, P, P, P, P, P, I, I, I, I, B, I]),
    "orc_bucket": (I, [I, I, I, P, P, P, P, P, P, P]),
    "orc_moe_gathered": (I, [I, P, P, P, P, P, P, P, I, I, I, I]),
}


class DS3Tensor(C.Structure):
    """Layout of the reference's ds3_tensor_t (src/ds3.h:233-241)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_int), ("n_dims", C.c_uint32),
                ("ne", C.c_uint64 * 4), ("nb", C.c_uint64 * 4), ("data", C.c_void_p), ("size", C.c_size_t)]


_REF = {
    "ds3_ref_dequantize_tensor": (P, [C.POINTER(DS3Tensor)]),
    "ds3_ref_dequantize_row": (I, [C.POINTER(DS3Tensor), I, P]),
    "ds3_ref_vec_matmul": (None, [P, P, P, I, I]),
    "ds3_ref_softmax": (None, [P, I]),
    "ds3_ref_topk": (None, [P, I, I, P, P]),
    "ds3_ref_silu": (None, [P, P, I]),
    "ds3_ref_mul": (None, [P, P, P, I]),
    "ds3_ref_add": (None, [P, P, P, I]),
    "ds3_ref_rms_norm": (None, [P, P, F, I, P]),
    "ds3_ref_matmul": (None, [P, P, P, I, I, I]),
    "ds3_ref_moe_ffn": (None, [P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, B]),
}

_orc = None
_ref = None
_libc = C.CDLL(None)
_libc.free.argtypes = [P]


def _bind(lib, table):
    for k, (r, a) in table.items():
        f = getattr(lib, k)
        f.restype, f.argtypes = r, a
    return lib


def orc():
    global _orc
    if _orc is None:
        if not ORACLE_SO.exists():
            subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), str(ORACLE_SO)], check=True)
        _orc = _bind(C.CDLL(str(ORACLE_SO)), _ORC)
    return _orc


def ref():
    """The compiled reference, or None where it was never built."""
    global _ref
    if _ref is None and REF_SO.exists():
        _ref = _bind(C.CDLL(str(REF_SO)), _REF)
    return _ref


def ptr(a: np.ndarray):
    return a.ctypes.data if a is not None else None


def dequantize(type_: int, raw: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    rc = orc().orc_dequantize(type_, ptr(raw), raw.nbytes, n, ptr(out))
    assert rc == 0, "oracle dequantize rejected the input"
    return out


def ref_dequantize(type_: int, raw: np.ndarray, n: int) -> np.ndarray:
    t = DS3Tensor()
    t.type, t.n_dims = type_, 1
    t.ne[0] = n
    t.data, t.size = raw.ctypes.data, raw.nbytes
    p = ref().ds3_ref_dequantize_tensor(C.byref(t))
    assert p, "reference dequantize rejected the input"
    out = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(n,)).copy()
    _libc.free(p)
    return out


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Rows of x normalised as src/ds3_reference.c:329-342 does (left-to-right sum of squares)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        orc().orc_rms_norm(ptr(x[r]), ptr(w), eps, x.shape[1], ptr(out[r]))
    return out


def vec_matmul(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    out_dim, in_dim = W.shape
    y = np.empty(out_dim, np.float32)
    orc().orc_vec_matmul(ptr(np.ascontiguousarray(x, np.float32)), ptr(np.ascontiguousarray(W, np.float32)),
                         ptr(y), in_dim, out_dim)
    return y


def route(logits: np.ndarray, k: int, norm: bool = True, with_probs: bool = False):
    """softmax -> top-k -> renorm of one token's logits (copy)."""
    lg = np.array(logits, np.float32)
    idx = np.empty(k, np.int32)
    sc = np.empty(k, np.float32)
    orc().orc_route(ptr(lg), lg.size, k, norm, ptr(idx), ptr(sc))
    return (idx, sc, lg) if with_probs else (idx, sc)


def moe_tokens(x: np.ndarray, wr: np.ndarray, wg: np.ndarray, wu: np.ndarray, wd: np.ndarray,
               n_expert: int, n_used: int, n_ff: int, threads: int = 8, norm: bool = True):
    """Per-token oracle MoE on FP32 weights: (out [T][E], idx [T][k], scores [T][k], probs [T][n_expert])."""
    T, K = x.shape
    out = np.empty((T, K), np.float32)
    logits = np.empty((T, n_expert), np.float32)
    sc = np.empty((T, n_used), np.float32)
    idx = np.empty((T, n_used), np.int32)
    rc = orc().orc_moe_ffn_tokens(T, ptr(x), ptr(wr), ptr(wg), ptr(wu), ptr(wd), ptr(out), ptr(logits), ptr(sc),
                                  ptr(idx), K, n_expert, n_used, n_ff, norm, threads)
    assert rc == 0
    return out, idx, sc, logits


def bucket(idx: np.ndarray, scores: np.ndarray, n_expert: int):
    T, k = idx.shape
    counts = np.empty(n_expert, np.int32)
    offsets = np.empty(n_expert, np.int32)
    ids = np.empty(T * k, np.int32)
    wts = np.empty(T * k, np.float32)
    pos = np.empty(T * k, np.int32)
    rc = orc().orc_bucket(T, k, n_expert, ptr(np.ascontiguousarray(idx, np.int32)),
                          ptr(np.ascontiguousarray(scores, np.float32)), ptr(counts), ptr(offsets), ptr(ids),
                          ptr(wts), ptr(pos))
    assert rc == 0
    return counts, offsets, ids, wts, pos


def gathered(x, idx, scores, wg, wu, wd, n_expert, n_ff):
    T, K = x.shape
    out = np.empty((T, K), np.float32)
    rc = orc().orc_moe_gathered(T, ptr(x), ptr(np.ascontiguousarray(idx, np.int32)),
                                ptr(np.ascontiguousarray(scores, np.float32)), ptr(wg), ptr(wu), ptr(wd), ptr(out),
                                K, n_expert, idx.shape[1], n_ff)
    assert rc == 0
    return out


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    return float(np.linalg.norm(a64 - b64) / max(np.linalg.norm(b64), 1e-30))
