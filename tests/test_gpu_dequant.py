"""GPU block decoders (ds3_hip_dequantize) against the oracle: bit-exact, on
random bytes (every scale/code pattern) and on generator-quantised weights."""
import numpy as np
import pytest

import _oracle as O
from qw3_amd import ds3
from qw3_amd import workload as W

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("t,per,nb", [(ds3.TYPE_Q4_K, 256, 144), (ds3.TYPE_Q6_K, 256, 210),
                                      (ds3.TYPE_Q8_0, 32, 34), (ds3.TYPE_F16, 1, 2), (ds3.TYPE_F32, 1, 4)])
def test_dequant_random_bytes(hip_ready, t, per, nb):
    rng = np.random.default_rng(t)
    n_blocks = 8192 if per > 1 else 1 << 17
    raw = rng.integers(0, 256, n_blocks * nb, dtype=np.uint8)
    n = n_blocks * per
    print(f"  dequant type={t} n={n}", flush=True)
    src = ds3.Buffer.from_array(raw)
    dst = ds3.Buffer.alloc(n * 4)
    ds3.dequantize(src, t, n, dst)
    got = dst.read(np.float32, n)
    want = O.dequantize(t, raw, n)
    same = (bits(got) == bits(want)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), f"{(~same).sum()} values differ"


@pytest.mark.parametrize("t", [ds3.TYPE_Q4_K, ds3.TYPE_Q6_K, ds3.TYPE_Q8_0])
def test_dequant_expert_matrix(hip_ready, t):
    """A full real-shape expert matrix (768 x 2048, or 2048 x 768 for Q6_K), bit-exact."""
    rows, cols = (2048, 768) if t == ds3.TYPE_Q6_K else (768, 2048)
    raw = W.quant_matrix(t, W.NORMAL, 1234, 500 + t, rows, cols, 0.0, 0.02)
    print(f"  dequant expert type={t} {rows}x{cols}", flush=True)
    src = ds3.Buffer.from_array(raw)
    dst = ds3.Buffer.alloc(rows * cols * 4)
    ds3.dequantize(src, t, rows * cols, dst)
    assert np.array_equal(bits(dst.read(np.float32, rows * cols)), bits(O.dequantize(t, raw, rows * cols)))


def test_dequant_odd_offsets(hip_ready):
    """Q6_K / Q8_0 blocks start on 2-byte boundaries inside rows; decode from
    every such alignment."""
    rng = np.random.default_rng(3)
    for t, nb, per in ((ds3.TYPE_Q6_K, 210, 256), (ds3.TYPE_Q8_0, 34, 32)):
        raw = rng.integers(0, 256, 64 * nb + 16, dtype=np.uint8)
        src = ds3.Buffer.from_array(raw)
        for off in (2, 6, 10, 14):
            n = 63 * per
            dst = ds3.Buffer.alloc(n * 4)
            ds3.dequantize(src, t, n, dst, src_offset=off)
            want = O.dequantize(t, raw[off:off + 63 * nb].copy(), n)
            got = dst.read(np.float32, n)
            same = (bits(got) == bits(want)) | (np.isnan(got) & np.isnan(want))
            assert same.all(), (t, off)
