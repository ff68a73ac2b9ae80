"""Shared GPU-test cases: a synthetic layer on host and device plus its FP32
dequantisation (via the oracle) and oracle outputs on the same inputs."""
from __future__ import annotations

import numpy as np

import _oracle as O
from qw3_amd import ds3
from qw3_amd import workload as W

TOL_MAX_ABS = 2e-3      # north-star bar on combined outputs
TOL_REL_L2 = 1e-3


class Case:
    def __init__(self, spec: W.LayerSpec, seed: int = 1234, layer: int = 0, router: np.ndarray | None = None,
                 host: W.HostLayer | None = None):
        """router (optional): F32 router rows [E][K] in place of the generated ones.
        host (optional): an already generated layer, whose device copy the
        caller holds (self.dev is then None)."""
        self.spec = spec
        self.host = host if host is not None else W.make_layer(spec, seed, layer)
        if router is not None:
            assert spec.router_type == ds3.TYPE_F32
            self.host.router = np.ascontiguousarray(router, np.float32).reshape(-1).view(np.uint8)
        self.dev = self.host.to_device() if host is None else None
        E, K, F = spec.n_expert, spec.n_embd, spec.n_ff
        self.wr = O.dequantize(spec.router_type, self.host.router, E * K).reshape(E, K)
        self.wg = O.dequantize(spec.gate_type, self.host.gate, E * F * K)
        self.wu = O.dequantize(spec.up_type, self.host.up, E * F * K)
        self.wd = O.dequantize(spec.down_type, self.host.down, E * K * F)

    def oracle(self, x: np.ndarray, n_used: int = W.N_USED, norm: bool = True, threads: int = 16):
        s = self.spec
        return O.moe_tokens(x, self.wr, self.wg, self.wu, self.wd, s.n_expert, n_used, s.n_ff, threads, norm)

    def gpu_batch(self, x: np.ndarray, n_used: int = W.N_USED, prefill_min: int | None = None,
                  residual: np.ndarray | None = None, norm: bool = True):
        s = self.spec
        T = x.shape[0]
        xb = ds3.Buffer.from_array(x)
        out = ds3.Buffer.alloc(T * s.n_embd * 4)
        idx = ds3.Buffer.alloc(T * n_used * 4)
        sc = ds3.Buffer.alloc(T * n_used * 4)
        lg = ds3.Buffer.alloc(T * s.n_expert * 4)
        rb = ds3.Buffer.from_array(residual) if residual is not None else None
        prev = ds3.set_prefill_min_tokens(prefill_min) if prefill_min else None
        try:
            ds3.moe_ffn_batch(xb, self.dev.router, s.router_type, self.dev.experts, out, T, s.n_expert, n_used,
                              residual=rb, logits=lg, indices=idx, scores=sc, norm=norm)
        finally:
            if prev is not None:
                ds3.set_prefill_min_tokens(prev)
        return (out.read(np.float32, (T, s.n_embd)), idx.read(np.int32, (T, n_used)),
                sc.read(np.float32, (T, n_used)), lg.read(np.float32, (T, s.n_expert)))


def assert_close(got: np.ndarray, want: np.ndarray, max_abs: float = TOL_MAX_ABS, rel_l2: float = TOL_REL_L2):
    err = float(np.abs(got.astype(np.float64) - want).max())
    rl = O.rel_l2(got, want)
    print(f"    max_abs={err:.3e} rel_l2={rl:.3e}", flush=True)
    assert err <= max_abs, f"max-abs {err:.3e} > {max_abs}"
    assert rl <= rel_l2, f"rel-L2 {rl:.3e} > {rel_l2}"
    return err, rl


def index_mismatches(got_idx: np.ndarray, want_idx: np.ndarray, probs: np.ndarray | None = None) -> int:
    """Rows whose selected experts (in order) differ from the oracle's and are
    not explained by a tie: with `probs` (the oracle's softmax probabilities),
    a row may differ only where the swapped experts' probabilities are equal
    to within 2 ulp -- the reference's own order there is a rounding accident
    of expf on (nearly) equal logits."""
    bad = np.nonzero((got_idx != want_idx).any(axis=1))[0]
    unexplained = 0
    for r in bad:
        tie = probs is not None
        if tie:
            p = probs[r]
            for a, b in zip(got_idx[r], want_idx[r]):
                if a != b and abs(float(p[a]) - float(p[b])) > 2 * float(np.spacing(max(p[a], p[b]))):
                    tie = False
                    break
        print(f"    row {r}: gpu {got_idx[r].tolist()} oracle {want_idx[r].tolist()}"
              f"{' (tie)' if tie else ''}", flush=True)
        unexplained += 0 if tie else 1
    return unexplained


def cert_bfac(K: int) -> float:
    """The certified router's bound factor for K-long logits: B = bfac * A
    bounds |reference logit - S|, S the exact sum of the reference's fp32
    products and A = sum_k |s_k| over their exact prefix sums.  The reference's
    k-th partial sum rounds once, by at most u |s^_k| (u = 2^-24), so its
    total error is at most u sum_k |s^_k| <= u A / (1 - K u); the remaining
    factors cover the device's own fp32 evaluation of A and fp64 sum."""
    u = 2.0 ** -24
    L = K / 256
    a_fac = (1 + u) / (1 - (L + 10) * u) / (1 - 2.01 * K * (3 * L + 14) * u)
    return (u / (1 - K * u) + (L + 10) * 2.0 ** -52) * a_fac


def cert_bound(x: np.ndarray, wr: np.ndarray) -> np.ndarray:
    """[T][E]: bfac * sum_k |s_k| from exact (fp64) prefix sums of the fp32
    products x[t][i] * wr[e][i]."""
    T, K = x.shape
    bfac = cert_bfac(K)
    out = np.empty((T, wr.shape[0]))
    for t in range(T):
        pr = (x[t][None, :] * wr).astype(np.float32).astype(np.float64)
        out[t] = bfac * np.abs(np.cumsum(pr, axis=1)).sum(axis=1)
    return out
