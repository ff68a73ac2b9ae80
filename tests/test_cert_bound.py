"""The error bound behind the certified router, checked on the CPU against
the reference's own sequential fp32 sums (src/ds3_reference.c:424-434, via
the oracle): |reference logit - S| <= bfac * A for every input, S the exact
sum of the reference's fp32 products and A the sum of |prefix sums|.  The
inputs include ones built to make the sequential sum's rounding errors
add up (equal positive products), where the bound must still hold and is
nearly reached, so a bound that drops a term or a factor fails here."""
import numpy as np
import pytest

import _oracle as O
from _cases import cert_bound


def _check(x: np.ndarray, wr: np.ndarray) -> float:
    ref = np.stack([O.vec_matmul(x[t], wr) for t in range(x.shape[0])]).astype(np.float64)
    S = np.stack([(x[t][None, :] * wr).astype(np.float32).astype(np.float64).sum(axis=1)
                  for t in range(x.shape[0])])
    B = cert_bound(x, wr)
    ratio = np.abs(ref - S) / B
    assert (ratio <= 1.0).all(), float(ratio.max())
    return float(ratio.max())


@pytest.mark.parametrize("K", [256, 2048, 4096])
def test_bound_random_router(K):
    rng = np.random.default_rng(K)
    wr = (rng.standard_normal((64, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((4, K)).astype(np.float32)
    r = _check(x, wr)
    assert r < 0.5


def test_bound_nearly_reached_by_aligned_rounding():
    """Equal positive products: every partial sum rounds the same way, the
    sequential error grows like u * sum |s_k|, and the bound is tight within
    a small factor."""
    K = 2048
    x = np.ones((1, K), np.float32)
    rows = []
    for c in (0.1, 1.0 / 3.0, 0.7, 1.1, 0.3333333):
        rows.append(np.full(K, c, np.float32))
    wr = np.stack(rows)
    r = _check(x, wr)
    print(f"max |err| / bound = {r:.3f}")
    assert r > 0.05


def test_bound_with_cancellation_and_bias():
    """Large cancelling terms and a final bias term (configuration 3's logit
    bias rides on the last element)."""
    K = 2048
    rng = np.random.default_rng(3)
    wr = (rng.standard_normal((32, K)) * 0.02).astype(np.float32)
    wr[:, : K // 2] += np.float32(5.0)
    wr[:, K // 2:] -= np.float32(5.0)
    wr[:, -1] = rng.normal(0, 4, 32).astype(np.float32)
    x = rng.standard_normal((3, K)).astype(np.float32)
    x[:, -1] = 1.0
    _check(x, wr)
