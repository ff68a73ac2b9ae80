"""Oracle restatement vs the reference's compiled ds3_reference.c on seeded
random inputs: every function on the path must agree bit for bit.  Skipped
where oracle/_ref was not built (it is built from the reference sources by
oracle/Makefile)."""
import numpy as np
import pytest

import _oracle as O
from qw3_amd import ds3

pytestmark = pytest.mark.skipif(O.ref() is None, reason="oracle/_ref/libds3ref.so not built")
RNG = np.random.default_rng(20261201)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("t,per,nb", [(ds3.TYPE_Q4_K, 256, 144), (ds3.TYPE_Q6_K, 256, 210),
                                      (ds3.TYPE_Q8_0, 32, 34), (ds3.TYPE_F16, 1, 2)])
def test_dequant_random_bytes(t, per, nb):
    # Arbitrary bytes: every scale / code / f16 pattern, incl. subnormal and non-finite scales.
    n_blocks = 4096 if per > 1 else 1 << 16
    raw = RNG.integers(0, 256, n_blocks * nb, dtype=np.uint8)
    got = O.dequantize(t, raw, n_blocks * per)
    want = O.ref_dequantize(t, raw, n_blocks * per)
    assert np.array_equal(bits(got), bits(want))


def test_dequant_rejects_like_reference():
    raw = np.zeros(144, np.uint8)
    out = np.empty(256, np.float32)
    assert O.orc().orc_dequantize(ds3.TYPE_Q4_K, O.ptr(raw), 143, 256, O.ptr(out)) == -1   # short buffer
    assert O.orc().orc_dequantize(ds3.TYPE_Q4_K, O.ptr(raw), 144, 255, O.ptr(out)) == -1   # not a block multiple
    assert O.orc().orc_dequantize(99, O.ptr(raw), 144, 256, O.ptr(out)) == -1              # unknown type


@pytest.mark.parametrize("in_dim,out_dim", [(1, 1), (7, 3), (256, 16), (2048, 128), (768, 64)])
def test_vec_matmul(in_dim, out_dim):
    x = RNG.standard_normal(in_dim).astype(np.float32)
    W = (RNG.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    a, b = np.empty(out_dim, np.float32), np.empty(out_dim, np.float32)
    O.orc().orc_vec_matmul(O.ptr(x), O.ptr(W), O.ptr(a), in_dim, out_dim)
    O.ref().ds3_ref_vec_matmul(O.ptr(x), O.ptr(W), O.ptr(b), in_dim, out_dim)
    assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("n,k", [(128, 8), (16, 4), (8, 8), (5, 1)])
def test_softmax_topk(n, k):
    for trial in range(20):
        v = RNG.standard_normal(n).astype(np.float32)
        if trial % 3 == 0:
            v[RNG.integers(0, n, n // 3)] = v[0]             # planted exact ties
        a, b = v.copy(), v.copy()
        O.orc().orc_softmax(O.ptr(a), n)
        O.ref().ds3_ref_softmax(O.ptr(b), n)
        assert np.array_equal(bits(a), bits(b))
        ia, ib = np.empty(k, np.int32), np.empty(k, np.int32)
        va, vb = np.empty(k, np.float32), np.empty(k, np.float32)
        O.orc().orc_topk(O.ptr(a), n, k, O.ptr(ia), O.ptr(va))
        O.ref().ds3_ref_topk(O.ptr(b), n, k, O.ptr(ib), O.ptr(vb))
        assert np.array_equal(ia, ib) and np.array_equal(bits(va), bits(vb))


def test_silu_mul_add_rmsnorm():
    n = 4099
    x = (RNG.standard_normal(n) * 4).astype(np.float32)
    y = RNG.standard_normal(n).astype(np.float32)
    for name, args in (("silu", 1), ("mul", 2), ("add", 2)):
        a, b = np.empty(n, np.float32), np.empty(n, np.float32)
        ins = (x,) if args == 1 else (x, y)
        getattr(O.orc(), "orc_" + name)(*[O.ptr(i) for i in ins], O.ptr(a), n)
        getattr(O.ref(), "ds3_ref_" + name)(*[O.ptr(i) for i in ins], O.ptr(b), n)
        assert np.array_equal(bits(a), bits(b)), name
    w = (1 + 0.02 * RNG.standard_normal(n)).astype(np.float32)
    a, b = np.empty(n, np.float32), np.empty(n, np.float32)
    O.orc().orc_rms_norm(O.ptr(x), O.ptr(w), 1e-6, n, O.ptr(a))
    O.ref().ds3_ref_rms_norm(O.ptr(x), O.ptr(w), 1e-6, n, O.ptr(b))
    assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("shape", [(256, 16, 4, 128), (512, 32, 8, 256)])
def test_moe_ffn(shape, norm):
    K, E, k, Fd = shape
    x = RNG.standard_normal(K).astype(np.float32)
    wr = (RNG.standard_normal((E, K)) * 0.05).astype(np.float32)
    wg = (RNG.standard_normal(E * Fd * K) * 0.05).astype(np.float32)
    wu = (RNG.standard_normal(E * Fd * K) * 0.05).astype(np.float32)
    wd = (RNG.standard_normal(E * K * Fd) * 0.05).astype(np.float32)
    res = []
    for lib, fn in ((O.orc(), "orc_moe_ffn"), (O.ref(), "ds3_ref_moe_ffn")):
        out, lg = np.empty(K, np.float32), np.empty(E, np.float32)
        sc, idx = np.empty(k, np.float32), np.empty(k, np.int32)
        getattr(lib, fn)(O.ptr(x), O.ptr(wr), O.ptr(wg), O.ptr(wu), O.ptr(wd), None, None, None, O.ptr(out),
                         O.ptr(lg), O.ptr(sc), O.ptr(idx), K, E, k, Fd, 0, norm)
        res.append((out, lg, sc, idx))
    (o1, l1, s1, i1), (o2, l2, s2, i2) = res
    assert np.array_equal(i1, i2)
    for a, b in ((o1, o2), (l1, l2), (s1, s2)):
        assert np.array_equal(bits(a), bits(b))


def test_moe_ffn_shared_expert():
    K, E, k, Fd, Fs = 256, 8, 2, 128, 384
    x = RNG.standard_normal(K).astype(np.float32)
    wr = (RNG.standard_normal((E, K)) * 0.05).astype(np.float32)
    w = [(RNG.standard_normal(n) * 0.05).astype(np.float32) for n in (E * Fd * K, E * Fd * K, E * K * Fd,
                                                                       Fs * K, Fs * K, K * Fs)]
    res = []
    for lib, fn in ((O.orc(), "orc_moe_ffn"), (O.ref(), "ds3_ref_moe_ffn")):
        out, lg = np.empty(K, np.float32), np.empty(E, np.float32)
        sc, idx = np.empty(k, np.float32), np.empty(k, np.int32)
        getattr(lib, fn)(O.ptr(x), O.ptr(wr), *[O.ptr(a) for a in w], O.ptr(out), O.ptr(lg), O.ptr(sc), O.ptr(idx),
                         K, E, k, Fd, Fs, True)
        res.append(out)
    assert np.array_equal(bits(res[0]), bits(res[1]))
