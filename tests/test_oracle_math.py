"""Pins of the oracle that do not come from the reference's code: brute
force, invariants and closed forms, chosen so a plausible slip (wrong nibble,
wrong index, dropped term) fails."""
import numpy as np
import pytest

import _oracle as O
from qw3_amd import ds3
from qw3_amd import workload as W

RNG = np.random.default_rng(7)


def test_fp16_decode_exhaustive():
    """Every one of the 65,536 binary16 patterns decodes to numpy's float16
    value, bit for bit: all of them through the oracle's F16 dequantisation
    (one call), and every 97th also through its scalar orc_fp16_to_fp32."""
    h = np.arange(1 << 16, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = O.dequantize(ds3.TYPE_F16, h.view(np.uint8), h.size)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    one = np.array([O.orc().orc_fp16_to_fp32(int(v)) for v in h[::97]], np.float32)
    same1 = (one.view(np.uint32) == want[::97].view(np.uint32)) | (np.isnan(one) & np.isnan(want[::97]))
    assert same1.all()


def test_q8_0_exactly_representable_roundtrip():
    """Values k*d with d a power of two and |k| <= 127 survive quantise->dequantise exactly."""
    d = np.float32(2.0 ** -7)
    k = RNG.integers(-127, 128, 32 * 64)
    k[::32] = 127                              # each block's max |k| is 127, so its scale is exactly d
    x = (k * d).astype(np.float32)
    raw = np.empty(64 * 34, np.uint8)
    from qw3_amd._native import gen
    assert gen().ds3gen_quantize(ds3.TYPE_Q8_0, x.ctypes.data, x.size, raw.ctypes.data) == raw.size
    assert np.array_equal(O.dequantize(ds3.TYPE_Q8_0, raw, x.size), x)


def test_q4k_dequant_closed_form():
    """Q4_K: each output equals d*sc*q - dmin*m rounded once to float32,
    with (sc, m) unpacked from the 12 scale bytes by bit arithmetic written
    here from the block layout, checked on random blocks."""
    nblk = 512
    raw = RNG.integers(0, 256, nblk * 144, dtype=np.uint8)
    raw = raw.reshape(nblk, 144)
    raw[:, 1] &= 0x3B                          # keep d, dmin finite and small
    raw[:, 3] &= 0x3B
    got = O.dequantize(ds3.TYPE_Q4_K, raw.reshape(-1), nblk * 256).reshape(nblk, 256)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dm = raw[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    s = raw[:, 4:16].astype(np.int64)
    sc = np.zeros((nblk, 8), np.int64)
    mn = np.zeros((nblk, 8), np.int64)
    sc[:, :4], mn[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = raw[:, 16:].astype(np.int64).reshape(nblk, 4, 32)
    q = np.concatenate([np.stack([qs[:, g] & 15, qs[:, g] >> 4], 1) for g in range(4)], 1)   # [nblk, 8, 32]
    want = (d[:, None, None] * sc[:, :, None] * q - dm[:, None, None] * mn[:, :, None]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.reshape(nblk, 256).view(np.uint32))


def test_topk_brute_force():
    for n, k in ((128, 8), (16, 4), (9, 9)):
        for _ in range(50):
            v = RNG.integers(-5, 6, n).astype(np.float32)      # many exact ties
            idx = np.empty(k, np.int32)
            val = np.empty(k, np.float32)
            assert O.orc().orc_topk(O.ptr(v), n, k, O.ptr(idx), O.ptr(val)) == 0
            order = sorted(range(n), key=lambda i: (-v[i], i))[:k]   # value desc, index asc
            assert idx.tolist() == order
            assert np.array_equal(val, v[order])


def test_route_invariants():
    for _ in range(20):
        lg = RNG.standard_normal(128).astype(np.float32)
        idx, sc = O.route(lg, 8, norm=True)
        assert len(set(idx.tolist())) == 8
        assert np.all(np.diff(sc) <= 0)                       # descending
        assert abs(float(sc.sum()) - 1.0) < 1e-6
        assert np.array_equal(np.sort(idx), np.sort(np.argsort(-lg, kind="stable")[:8]))
        idx2, sc2 = O.route(lg, 8, norm=False)
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        assert np.allclose(sc2, p[idx2], rtol=1e-6, atol=0)


def test_bucket_invariants_and_brute_force():
    T, k, E = 300, 8, 128
    idx = np.stack([RNG.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    sc = RNG.random((T, k)).astype(np.float32)
    counts, offsets, ids, wts, pos = O.bucket(idx, sc, E)
    assert counts.sum() == T * k
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)[:-1]]))
    for e in range(E):
        lst = ids[offsets[e]:offsets[e] + counts[e]]
        assert np.array_equal(lst, np.nonzero((idx == e).any(1))[0])     # token order
    t_of = np.repeat(np.arange(T), k)
    assert np.array_equal(ids[pos], t_of)                                # round trip
    assert np.array_equal(wts[pos], sc.reshape(-1))
    bad = idx.copy()
    bad[3, 2] = E
    assert O.orc().orc_bucket(T, k, E, O.ptr(bad), O.ptr(sc), O.ptr(counts), O.ptr(offsets), O.ptr(ids),
                              O.ptr(wts), O.ptr(pos)) == -1


def test_gathered_equals_per_token():
    """The gathered prefill order (expert-major) equals the per-token oracle
    up to float rounding of the different summation order."""
    K, E, k, Fd, T = 256, 16, 4, 128, 40
    x = RNG.standard_normal((T, K)).astype(np.float32)
    wr = (RNG.standard_normal((E, K)) * 0.05).astype(np.float32)
    wg, wu, wd = [(RNG.standard_normal(E * Fd * K) * 0.05).astype(np.float32) for _ in range(3)]
    out, idx, sc, _ = O.moe_tokens(x, wr, wg, wu, wd, E, k, Fd)
    g = O.gathered(x, idx, sc, wg, wu, wd, E, Fd)
    assert O.rel_l2(g, out) < 1e-6


def test_moe_identical_experts_closed_form():
    """With every expert identical and renormalised weights, the output is
    that one expert's FFN (weights sum to 1), whatever the routing."""
    K, E, k, Fd = 256, 16, 4, 128
    x = RNG.standard_normal((3, K)).astype(np.float32)
    wr = (RNG.standard_normal((E, K)) * 0.05).astype(np.float32)
    one = [(RNG.standard_normal(n) * 0.05).astype(np.float32) for n in (Fd * K, Fd * K, K * Fd)]
    wg, wu, wd = [np.tile(a, E) for a in one]
    out, _, _, _ = O.moe_tokens(x, wr, wg, wu, wd, E, k, Fd)
    g = x.astype(np.float64) @ one[0].reshape(Fd, K).T.astype(np.float64)
    u = x.astype(np.float64) @ one[1].reshape(Fd, K).T.astype(np.float64)
    h = g / (1 + np.exp(-g)) * u
    y = h @ one[2].reshape(K, Fd).T.astype(np.float64)
    assert O.rel_l2(out, y) < 1e-5


def test_planted_mistake_is_caught():
    """A swapped low/high nibble in the Q4_K decode (a plausible slip) breaks
    the reference's known answer, so the KAT above would fail it."""
    import json
    from pathlib import Path
    kat = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())["dequant"][0]
    raw = np.array(kat["bytes"], np.uint8)
    swapped = raw.copy()
    qs = swapped[16:]
    swapped[16:] = ((qs & 15) << 4) | (qs >> 4)
    got = O.dequantize(ds3.TYPE_Q4_K, swapped, 256)
    assert got[0] != kat["expect"]["0"]
