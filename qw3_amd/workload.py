"""Synthetic Qwen3-30B-A3B MoE-FFN workloads (the configurations benchmarked).

All values come from the counter-based generator in libds3gen.so, so a
(seed, layer, tensor) triple always produces the same bytes.  Expert weights
are drawn N(0, 0.02) in FP32 and quantised with this project's GGUF block
quantisers; the router stays FP32 (or Q8_0 for the Q8_0 sweep).

Configurations (numbering of the benchmark brief):
  1  T=1 decode: x = RMSNorm(z, 1 + N(0, 0.02)), z ~ N(0, 1); router N(0, 0.02)
  2  T=512 prefill: x ~ N(0, 1); router U(-a, a), a = 0.02*sqrt(3)
  3  T=2048 skewed: as 2 plus a per-expert logit bias b_e = beta*ln(p_e),
     p_e ~ rank_e^-1.2 over a seeded permutation, injected exactly through the
     input: x[:, n_embd-1] = 1 and router[e][n_embd-1] = b_e
  4  48-layer decode stack: 48 independent layers, h <- h + MoE_l(h)
  5  Q8_0 sweep: every expert matrix and the router in Q8_0
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

from . import ds3
from ._native import gen

N_EMBD, N_FF, N_EXPERT, N_USED = 2048, 768, 128, 8
NORMAL, UNIFORM = 0, 1
K_X, K_ROUTER, K_GATE, K_UP, K_DOWN, K_GAIN, K_PERM = range(7)


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def stream_id(layer: int, kind: int) -> int:
    return (layer << 8) | kind


def fill(dist: int, seed: int, stream: int, n: int, a: float, b: float, offset: int = 0) -> np.ndarray:
    out = np.empty(n, np.float32)
    gen().ds3gen_fill(dist, seed, stream, offset, n, a, b, out.ctypes.data)
    return out


def quant_matrix(type_: int, dist: int, seed: int, stream: int, rows: int, cols: int, a: float, b: float) -> np.ndarray:
    """[rows][cols] values quantised row by row -> raw GGUF bytes."""
    rb = ds3.row_bytes(type_, cols)
    buf = np.empty(rows * rb, np.uint8)
    rc = gen().ds3gen_matrix(type_, dist, seed, stream, rows, cols, a, b, buf.ctypes.data, _threads())
    if rc != 0:
        raise RuntimeError("ds3gen_matrix failed")
    return buf


def fp16_bits(x: float) -> int:
    return int(gen().ds3gen_fp32_to_fp16(C.c_float(x)))


@dataclass
class LayerSpec:
    gate_type: int = ds3.TYPE_Q4_K
    up_type: int = ds3.TYPE_Q4_K
    down_type: int = ds3.TYPE_Q6_K
    router_type: int = ds3.TYPE_F32
    router_dist: int = NORMAL           # NORMAL: N(0, std); UNIFORM: U(-std*sqrt3, std*sqrt3)
    std: float = 0.02
    n_embd: int = N_EMBD
    n_ff: int = N_FF
    n_expert: int = N_EXPERT
    zipf_beta: float = 0.0              # > 0: config-3 logit bias through the last input coordinate
    zipf_s: float = 1.2


@dataclass
class HostLayer:
    spec: LayerSpec
    router: np.ndarray                  # raw bytes (F32 or Q8_0) [n_expert][n_embd]
    gate: np.ndarray                    # raw bytes [n_expert*n_ff][n_embd]
    up: np.ndarray
    down: np.ndarray                    # raw bytes [n_expert*n_embd][n_ff]
    bias: np.ndarray | None = None

    def to_device(self, readonly: bool = False) -> "DeviceLayer":
        """readonly: import every tensor as the engine imports mmap'd GGUF
        weights (ds3_hip_buffer_from_mmap); otherwise plain device buffers."""
        s = self.spec
        put = ds3.Buffer.from_mmap_array if readonly else ds3.Buffer.from_array
        return DeviceLayer(
            spec=s,
            router=put(self.router),
            experts=ds3.ExpertTensors(put(self.gate), put(self.up), put(self.down), s.gate_type, s.up_type,
                                      s.down_type, s.n_embd, s.n_ff))


@dataclass
class DeviceLayer:
    spec: LayerSpec
    router: ds3.Buffer
    experts: ds3.ExpertTensors
    extra: dict = field(default_factory=dict)


def zipf_bias(seed: int, layer: int, n_expert: int, s: float, beta: float) -> np.ndarray:
    """b_e = beta * ln(p_e), p_e proportional to rank_e^-s, ranks a seeded permutation."""
    keys = fill(UNIFORM, seed, stream_id(layer, K_PERM), n_expert, 0.0, 1.0)
    rank = np.empty(n_expert, np.int64)
    rank[np.argsort(keys, kind="stable")] = np.arange(1, n_expert + 1)
    p = rank.astype(np.float64) ** (-s)
    p /= p.sum()
    return (beta * np.log(p)).astype(np.float32)


def make_layer(spec: LayerSpec, seed: int = 1234, layer: int = 0) -> HostLayer:
    E, K, F = spec.n_expert, spec.n_embd, spec.n_ff
    if spec.router_dist == UNIFORM:
        a = spec.std * np.sqrt(3.0)
        rdist, ra, rb_ = UNIFORM, -a, a
    else:
        rdist, ra, rb_ = NORMAL, 0.0, spec.std
    bias = None
    if spec.router_type == ds3.TYPE_F32:
        router = fill(rdist, seed, stream_id(layer, K_ROUTER), E * K, ra, rb_).reshape(E, K)
        if spec.zipf_beta > 0:
            bias = zipf_bias(seed, layer, E, spec.zipf_s, spec.zipf_beta)
            router[:, K - 1] = bias
        router = router.view(np.uint8).reshape(-1)
    else:
        if spec.zipf_beta > 0:
            raise ValueError("the Zipf bias needs an F32 router")
        router = quant_matrix(spec.router_type, rdist, seed, stream_id(layer, K_ROUTER), E, K, ra, rb_)
    gate = quant_matrix(spec.gate_type, NORMAL, seed, stream_id(layer, K_GATE), E * F, K, 0.0, spec.std)
    up = quant_matrix(spec.up_type, NORMAL, seed, stream_id(layer, K_UP), E * F, K, 0.0, spec.std)
    down = quant_matrix(spec.down_type, NORMAL, seed, stream_id(layer, K_DOWN), E * K, F, 0.0, spec.std)
    return HostLayer(spec, router, gate, up, down, bias)


def rms_norm(z: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Input preparation of config 1 (reference src/ds3_reference.c:329-342, float32)."""
    z = z.astype(np.float32)
    ss = np.float32(np.mean(z.astype(np.float64) ** 2)) + np.float32(eps)
    return (z * (np.float32(1.0) / np.sqrt(ss)) * w).astype(np.float32)


def make_inputs(config: int, T: int, seed: int = 1234, layer: int = 0, step: int = 0,
                n_embd: int = N_EMBD) -> np.ndarray:
    """Token inputs [T][n_embd] f32 for a configuration; `step` selects fresh rows."""
    st = stream_id(layer, K_X)
    off = step * T * n_embd
    if config == 1:
        z = fill(NORMAL, seed, st, T * n_embd, 0.0, 1.0, off).reshape(T, n_embd)
        gain = 1.0 + fill(NORMAL, seed, stream_id(layer, K_GAIN), n_embd, 0.0, 0.02)
        return np.stack([rms_norm(z[t], gain) for t in range(T)]).astype(np.float32)
    x = fill(NORMAL, seed, st, T * n_embd, 0.0, 1.0, off).reshape(T, n_embd)
    if config == 3:
        x[:, n_embd - 1] = 1.0
    return x


def config_spec(config: int) -> LayerSpec:
    if config in (1, 4):
        return LayerSpec()
    if config == 2:
        return LayerSpec(router_dist=UNIFORM)
    if config == 3:
        return LayerSpec(router_dist=UNIFORM, zipf_beta=1.0)
    if config == 5:
        return LayerSpec(ds3.TYPE_Q8_0, ds3.TYPE_Q8_0, ds3.TYPE_Q8_0, ds3.TYPE_Q8_0)
    raise ValueError(config)


def expert_bytes(spec: LayerSpec) -> int:
    """Quantised bytes of one expert (gate + up + down)."""
    return spec.n_ff * (ds3.row_bytes(spec.gate_type, spec.n_embd) + ds3.row_bytes(spec.up_type, spec.n_embd)) + \
        spec.n_embd * ds3.row_bytes(spec.down_type, spec.n_ff)


def router_bytes(spec: LayerSpec) -> int:
    return spec.n_expert * ds3.row_bytes(spec.router_type, spec.n_embd)


def algorithmic_bytes(spec: LayerSpec, T: int, distinct_experts: int) -> int:
    """HBM bytes one layer call must move: distinct selected experts' weights,
    the router, x read and y write."""
    return distinct_experts * expert_bytes(spec) + router_bytes(spec) + 2 * T * spec.n_embd * 4


def algorithmic_flops(spec: LayerSpec, T: int, n_used: int = N_USED) -> int:
    return T * (2 * spec.n_expert * spec.n_embd + n_used * 3 * 2 * spec.n_ff * spec.n_embd)
