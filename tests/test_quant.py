"""This project's GGUF quantisers and generator (qw3_amd/csrc/gen).

The reference ships no usable quantiser, so quantisation itself is
"parity unpinned" by design: parity is defined on the quantised bytes, which
GPU and oracle both decode.  These tests bound the round-trip error (via the
oracle's decoder) and pin the helpers that have an exact answer."""
import numpy as np
import pytest

import _oracle as O
from qw3_amd import ds3
from qw3_amd import workload as W
from qw3_amd._native import gen


def test_fp32_to_fp16_matches_numpy_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-8, 1e-5, 1e-2, 1, 100, 7e4)])
    x = np.concatenate([x, np.float32([0.0, -0.0, 65504, 65520, 65519.99, np.inf, -np.inf, 5.96e-8, 2.98e-8])])
    got = np.array([gen().ds3gen_fp32_to_fp16(float(v)) for v in x], np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_generator_is_deterministic_and_split_invariant():
    a = W.fill(W.NORMAL, 5, 11, 10000, 0.0, 1.0)
    b = np.concatenate([W.fill(W.NORMAL, 5, 11, 3000, 0.0, 1.0), W.fill(W.NORMAL, 5, 11, 7000, 0.0, 1.0, 3000)])
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 0.05 and abs(a.std() - 1) < 0.05
    u = W.fill(W.UNIFORM, 5, 12, 10000, -2.0, 2.0)
    assert u.min() >= -2 and u.max() < 2 and abs(u.mean()) < 0.1
    assert not np.array_equal(a, W.fill(W.NORMAL, 5, 12, 10000, 0.0, 1.0))


@pytest.mark.parametrize("t,rmse_max", [(ds3.TYPE_Q8_0, 0.012), (ds3.TYPE_Q6_K, 0.04), (ds3.TYPE_Q4_K, 0.13)])
def test_roundtrip_error(t, rmse_max):
    rows, cols, std = 64, 2048, 0.02
    raw = W.quant_matrix(t, W.NORMAL, 3, 40 + t, rows, cols, 0.0, std)
    x = W.fill(W.NORMAL, 3, 40 + t, rows * cols, 0.0, std)
    y = O.dequantize(t, raw, rows * cols)
    err = y - x
    assert np.sqrt(np.mean(err ** 2)) / std < rmse_max
    # no block is badly off (a packing slip shows up as errors ~ the signal)
    per, _ = ds3.BLOCK[t]
    blk_err = np.abs(err.reshape(-1, per)).max(1)
    blk_amp = np.abs(x.reshape(-1, per)).max(1)
    assert np.all(blk_err <= 0.2 * blk_amp + 1e-9)


def test_zero_input_quantises_to_zero():
    for t in (ds3.TYPE_Q8_0, ds3.TYPE_Q6_K, ds3.TYPE_Q4_K):
        x = np.zeros(512, np.float32)
        raw = np.empty(ds3.row_bytes(t, 512), np.uint8)
        gen().ds3gen_quantize(t, x.ctypes.data, 512, raw.ctypes.data)
        assert np.all(O.dequantize(t, raw, 512) == 0)


def test_thread_count_does_not_change_bytes():
    r1 = np.empty(32 * 144 * 8, np.uint8)
    r2 = np.empty_like(r1)
    assert gen().ds3gen_matrix(ds3.TYPE_Q4_K, 0, 9, 9, 32, 2048, 0.0, 0.02, r1.ctypes.data, 1) == 0
    assert gen().ds3gen_matrix(ds3.TYPE_Q4_K, 0, 9, 9, 32, 2048, 0.0, 0.02, r2.ctypes.data, 7) == 0
    assert np.array_equal(r1, r2)
