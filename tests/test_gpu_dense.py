"""Dense quantised products on the GPU (the engine's attention projections and
output head, reference src/ds3_engine.c:181-271), through the C ABI, against
the oracle's FP32 dequantisation of the same bytes.

Bars:
  - the fp32 paths (vec_matmul_*, matmul_quantized_batch below the MFMA row
    count, vec_matmul_q4k_half): max-abs 1e-4, the reference's own tolerance
    (tests/test_matmul_quant_metal.c:66);
  - the fp16-MFMA path of matmul_quantized_batch: the north-star bar on
    outputs, relative L2 <= 1e-3, and max-abs <= 2e-3 on outputs scaled to
    unit RMS."""
import numpy as np
import pytest

import _oracle as O
from qw3_amd import ds3
from qw3_amd import workload as W
from qw3_amd._native import hip

pytestmark = pytest.mark.gpu

HEAD_N = 151936          # Qwen3 vocabulary (reference src/ds3.h:75), the output head's rows
TOL_FP32 = 1e-4
MFMA_REL_L2 = 1e-3
MFMA_MAX_ABS_UNIT_RMS = 2e-3


def normal_matrix(t, seed, rows, cols):
    """Weights quantised from N(0, 0.02), as the configs' expert weights."""
    return W.quant_matrix(t, W.NORMAL, seed, t, rows, cols, 0.0, 0.02)


def kernels_run():
    return set(ds3.kernel_stats())


@pytest.mark.parametrize("t,M,N,K", [(12, 64, 512, 2048), (12, 512, 4096, 2048), (14, 100, 2048, 4096),
                                     (8, 512, 512, 2048), (14, 77, 256, 512)])
def test_matmul_quantized_batch_mfma(hip_ready, t, M, N, K):
    """From 64 rows of A, Q4_K / Q6_K / Q8_0 products with K % 512 == 0 and
    N % 256 == 0 run on the matrix cores (fp16 operands); ragged M, a weight
    offset inside the buffer and both halves of W's rows are covered."""
    rng = np.random.default_rng(M + N + K + t)
    A = rng.standard_normal((M, K)).astype(np.float32)
    raw = normal_matrix(t, 5, N, K)
    Wf = O.dequantize(t, raw, N * K).reshape(N, K).astype(np.float64)
    want = A.astype(np.float64) @ Wf.T
    off = 768
    wb = ds3.Buffer.alloc(raw.nbytes + off)
    wb.write(raw, offset=off)
    cb = ds3.Buffer.alloc(M * N * 4)
    print(f"  dense MFMA {ds3.TYPE_NAMES[t]} M={M} N={N} K={K}", flush=True)
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing(1)
    rc = hip().ds3_hip_matmul_quantized_batch(ds3.Buffer.from_array(A), wb, cb, M, N, K, ds3.row_bytes(t, K), off, t)
    hip().ds3_hip_kernel_timing(0)
    assert rc == 0
    assert "dense_mfma" in kernels_run()              # the matrix-core path served the call
    got = cb.read(np.float32, (M, N)).astype(np.float64)
    rms = float(np.sqrt(np.mean(want ** 2)))
    rl = O.rel_l2(got, want)
    ma = float(np.abs(got - want).max()) / rms
    print(f"    rel_l2={rl:.2e} max_abs/rms={ma:.2e}", flush=True)
    assert rl <= MFMA_REL_L2
    assert ma <= MFMA_MAX_ABS_UNIT_RMS


def test_matmul_quantized_batch_paths(hip_ready):
    """The row count switch: below it the fp32 path (the reference's own
    tolerance), from it the MFMA path; ds3_hip_set_dense_mfma_min_rows moves it."""
    t, N, K = 12, 512, 2048
    rng = np.random.default_rng(9)
    raw = normal_matrix(t, 6, N, K)
    Wf = O.dequantize(t, raw, N * K).reshape(N, K)
    wb = ds3.Buffer.from_array(raw)
    prev = hip().ds3_hip_set_dense_mfma_min_rows(0)
    try:
        for M, min_rows, path in ((32, 0, "gemv"), (64, 0, "dense_mfma"), (64, 65, "gemv"), (16, 16, "dense_mfma")):
            hip().ds3_hip_set_dense_mfma_min_rows(min_rows)
            A = rng.standard_normal((M, K)).astype(np.float32)
            want = np.stack([O.vec_matmul(A[m], Wf) for m in range(M)])
            cb = ds3.Buffer.alloc(M * N * 4)
            hip().ds3_hip_kernel_timing_reset()
            hip().ds3_hip_kernel_timing(1)
            assert hip().ds3_hip_matmul_quantized_batch(ds3.Buffer.from_array(A), wb, cb, M, N, K,
                                                        ds3.row_bytes(t, K), 0, t) == 0
            hip().ds3_hip_kernel_timing(0)
            ran = kernels_run()
            print(f"  M={M} min_rows={min_rows}: {sorted(ran)}", flush=True)
            assert path in ran
            got = cb.read(np.float32, (M, N))
            if path == "gemv":
                assert float(np.abs(got - want).max()) < TOL_FP32
            else:
                assert O.rel_l2(got, want) <= MFMA_REL_L2
    finally:
        hip().ds3_hip_set_dense_mfma_min_rows(prev)


SIMD_NAME = {12: "q4k", 14: "q6k", 8: "q8_0"}


def vec_matmul_kernel(t, xb, wb, yb, K, N, stride):
    """One vec_matmul call with kernel timing on; returns the kernels it ran."""
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing(1)
    rc = hip().ds3_hip_vec_matmul_quantized(xb, wb, yb, K, N, stride, t)
    hip().ds3_hip_kernel_timing(0)
    assert rc == 0
    return kernels_run()


@pytest.mark.parametrize("t,N,K", [(12, 1031, 2048), (14, 4099, 4096), (8, 333, 4096), (8, 16, 2048),
                                   (14, 1, 2048), (12, 17, 4096), (14, 40, 2048), (8, 9, 4096)])
def test_vec_matmul_one_token_path(hip_ready, t, N, K):
    """One token against dense, 16-byte aligned Q4_K / Q6_K / Q8_0 rows of
    K = 2048 or 4096 runs on the chunked one-token kernel (gemv1): row counts
    that leave a partial last chunk, a single row, and fewer rows than one
    chunk; the reference's tolerance, 1e-4 (tests/test_matmul_quant_metal.c:66)."""
    x = np.random.default_rng(N + K).standard_normal(K).astype(np.float32)
    raw = normal_matrix(t, 11, N, K)
    want = O.vec_matmul(x, O.dequantize(t, raw, N * K).reshape(N, K))
    yb = ds3.Buffer.alloc(N * 4)
    print(f"  gemv1 {ds3.TYPE_NAMES[t]} N={N} K={K}", flush=True)
    ran = vec_matmul_kernel(t, ds3.Buffer.from_array(x), ds3.Buffer.from_array(raw), yb, K, N, ds3.row_bytes(t, K))
    assert "gemv1" in ran and "gemv" not in ran
    err = float(np.abs(yb.read(np.float32, N) - want).max())
    print(f"    max_abs={err:.2e}", flush=True)
    assert err < TOL_FP32


def test_vec_matmul_one_token_fallbacks(hip_ready):
    """Rows the chunked kernel does not take go to the general kernel, with
    the same results: a weight base 8 bytes past a 16-byte boundary, rows
    padded past their bytes, and K outside {2048, 4096}."""
    t, N, K = 14, 300, 2048
    rb = ds3.row_bytes(t, K)
    rng = np.random.default_rng(5)
    x = rng.standard_normal(K).astype(np.float32)
    raw = normal_matrix(t, 12, N, K)
    want = O.vec_matmul(x, O.dequantize(t, raw, N * K).reshape(N, K))
    xb, yb = ds3.Buffer.from_array(x), ds3.Buffer.alloc(N * 4)
    # base 8 bytes off
    big = ds3.Buffer.alloc(raw.nbytes + 8)
    big.write(raw, offset=8)
    ran = vec_matmul_kernel(t, xb, big.view(8, raw.nbytes), yb, K, N, rb)
    assert "gemv" in ran and "gemv1" not in ran
    assert float(np.abs(yb.read(np.float32, N) - want).max()) < TOL_FP32
    # padded rows: 32 spare bytes per row
    pad = np.zeros((N, rb + 32), np.uint8)
    pad[:, :rb] = raw.reshape(N, rb)
    yb.zero()
    ran = vec_matmul_kernel(t, xb, ds3.Buffer.from_array(pad), yb, K, N, rb + 32)
    assert "gemv" in ran and "gemv1" not in ran
    assert float(np.abs(yb.read(np.float32, N) - want).max()) < TOL_FP32
    # K = 1024
    K2 = 1024
    raw2 = normal_matrix(t, 13, N, K2)
    want2 = O.vec_matmul(x[:K2], O.dequantize(t, raw2, N * K2).reshape(N, K2))
    ran = vec_matmul_kernel(t, ds3.Buffer.from_array(x[:K2]), ds3.Buffer.from_array(raw2), yb, K2, N,
                            ds3.row_bytes(t, K2))
    assert "gemv" in ran and "gemv1" not in ran
    assert float(np.abs(yb.read(np.float32, N) - want2).max()) < TOL_FP32


@pytest.mark.parametrize("t", [14, 8])
def test_output_head_vec_matmul(hip_ready, t):
    """The engine's output projection (dispatch_output_matmul, reference
    src/ds3_engine.c:212-247): 2048 -> 151,936 logits, Q6_K (Qwen3 Q4_K_M) and
    Q8_0 weights, through vec_matmul_quantized and the _simd name."""
    K = 2048
    x = np.random.default_rng(t).standard_normal(K).astype(np.float32)
    print(f"  head {ds3.TYPE_NAMES[t]} {HEAD_N} x {K}: generating", flush=True)
    raw = normal_matrix(t, 7, HEAD_N, K)
    want = O.vec_matmul(x, O.dequantize(t, raw, HEAD_N * K).reshape(HEAD_N, K))
    wb = ds3.Buffer.from_array(raw)
    xb = ds3.Buffer.from_array(x)
    yb = ds3.Buffer.alloc(HEAD_N * 4)
    rs = ds3.row_bytes(t, K)
    assert "gemv1" in vec_matmul_kernel(t, xb, wb, yb, K, HEAD_N, rs)      # the one-token chunked kernel
    err = float(np.abs(yb.read(np.float32, HEAD_N) - want).max())
    print(f"    max_abs={err:.2e}", flush=True)
    assert err < TOL_FP32
    simd = SIMD_NAME[t]
    yb.zero()
    assert getattr(hip(), f"ds3_hip_vec_matmul_{simd}_simd")(xb, wb, yb, K, HEAD_N, rs) == 0
    assert float(np.abs(yb.read(np.float32, HEAD_N) - want).max()) < TOL_FP32
    assert int(np.argmax(yb.read(np.float32, HEAD_N))) == int(np.argmax(want))


def test_vec_matmul_q4k_half(hip_ready):
    """reference src/ds3_metal.h:142-146: an fp16 input vector; the product is
    the fp32 one of the same values (tests/test_matmul_quant_metal.c's half
    case, tolerance 1e-4)."""
    K, N = 2048, 1024
    rng = np.random.default_rng(3)
    x16 = (rng.random(K) - 0.5).astype(np.float16)
    raw = W.quant_matrix(12, W.UNIFORM, 8, 12, N, K, -0.5, 0.5)
    want = O.vec_matmul(x16.astype(np.float32), O.dequantize(12, raw, N * K).reshape(N, K))
    yb = ds3.Buffer.alloc(N * 4)
    xb = ds3.Buffer.alloc(K * 2)
    xb.write(x16.view(np.uint8))
    assert hip().ds3_hip_vec_matmul_q4k_half(xb, ds3.Buffer.from_array(raw), yb, K, N, ds3.row_bytes(12, K)) == 0
    assert float(np.abs(yb.read(np.float32, N) - want).max()) < TOL_FP32
    # argument rules: in_dim % 256, short row stride, short x
    assert hip().ds3_hip_vec_matmul_q4k_half(xb, ds3.Buffer.from_array(raw), yb, K - 32, N, 1152) == -1
    assert hip().ds3_hip_vec_matmul_q4k_half(xb, ds3.Buffer.from_array(raw), yb, K, N, 1000) == -1
    assert hip().ds3_hip_vec_matmul_q4k_half(xb.view(0, K), ds3.Buffer.from_array(raw), yb, K, N, 1152) == -1
