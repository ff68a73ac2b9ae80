"""MoE-FFN throughput on one MI355X (benchmark contract: one JSON line on stdout).

Headline workload: one Qwen3-30B-A3B MoE-FFN layer
call on T = 512 tokens -- router, softmax/top-8, bucketing, grouped Q4_K
gate/up and Q6_K down products, SwiGLU and the weighted combine -- through the
C ABI (ds3_hip_moe_ffn_batch).  A step is one layer call on one batch; the
engine's output zeroing (reference src/ds3_engine.c:902) is part of the step.
Layers are cycled from `--layers` distinct resident copies so weights cannot
stay in the 256 MB Infinity Cache between steps.

The default run also measures every other configuration of BASELINE.json and
puts each under its own key of the same line:
  t1  configs[0]  T = 1 decode of the same layer shape
  c3  configs[2]  T = 2048, Zipf-skewed routing (the MFMA-bound configuration)
  c4  configs[3]  one token per step through 48 resident layers (HIP graph)
  c5  configs[4]  all-Q8_0 layer, T in {1, 4, 16, 64, 256, 1024}, on the GEMV
                  path and the grouped-MFMA path, with the crossover
  dense           the engine's dense products beside the MoE: the output head
                  GEMV (Q6_K, Q8_0) and a 512-row prefill projection (Q4_K)

roofline: the dominant kernel's algorithmic bytes per launch / its mean
duration, timed with HIP events on the library stream over a second pass of
the same steps (the timed region itself carries no per-kernel events).
cpu_baseline: the reference's own ds3_ref_moe_ffn (compiled from its sources
into oracle/_ref) on the host cores, FP32-dequantised weights resident, on a
bounded sample of the same workload; a 1-core pinned figure sits beside the
multi-thread one.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
FP16_PEAK_TFLOPS = 2500.0      # dense fp16 MFMA
C5_TOKENS = (1, 4, 8, 16, 32, 64, 256, 1024)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=100,
                   help="untimed steps enqueued back to back right before each timed region")
    p.add_argument("--tokens", type=int, default=None, help="tokens per step of a --config 2/3/5 run")
    p.add_argument("--layers", type=int, default=8, help="distinct resident layers cycled per step")
    p.add_argument("--config", type=int, default=0, choices=(0, 2, 3, 4, 5),
                   help="0 (default): every configuration in one line; 2, 3, 5: one layer on --tokens tokens "
                        "(+ T=1 under t1 for 2); 4: the decode stack alone")
    p.add_argument("--stack-layers", type=int, default=48, help="config 4: resident layers per decode step")
    p.add_argument("--stack-steps", type=int, default=200)
    p.add_argument("--no-graph", action="store_true",
                   help="configs 4 and the T=1 leg: enqueue every call eagerly instead of replaying captured HIP graphs")
    p.add_argument("--stack-block", action="store_true",
                   help="config 4: run each layer as the engine's FFN block (RMSNorm + MoE + residual)")
    p.add_argument("--t1-steps", type=int, default=1008)
    p.add_argument("--t1-zero", action="store_true",
                   help="T=1 leg: zero the output before every call (default: each call accumulates into the "
                        "output, the decode residual stream, with no zeroing launch)")
    p.add_argument("--no-t1", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--skip", type=str, default="",
                   help="default run: comma-separated legs to leave out (c3,c4,c5,dense)")
    p.add_argument("--cpu-tokens", type=int, default=512)
    p.add_argument("--copy-mib", type=int, default=0,
                   help="first run a plain device copy of this many MiB (k_copy, three times): the known-size "
                        "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    p.add_argument("--traffic", type=str, default=None,
                   help="JSON {kernel: HBM bytes per launch} from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs "
                        "(default: profiles/hbm_traffic.json)")
    return p.parse_args()


def kernel_bytes(name, spec, T, counts, n_used):
    """Algorithmic HBM bytes of one launch of `name` (per-kernel split of the
    layer's algorithmic bytes; see DESIGN.md, Measurement)."""
    from qw3_amd import ds3
    from qw3_amd import workload as W
    E, K, F = spec.n_expert, spec.n_embd, spec.n_ff
    distinct = int((counts > 0).sum())
    gu = F * (ds3.row_bytes(spec.gate_type, K) + ds3.row_bytes(spec.up_type, K))
    dn = K * ds3.row_bytes(spec.down_type, F)
    S = T * n_used
    # certified routing (T <= 16): the gate/up launch also streams the router
    # rows of every selected expert for the exact logits of the weights
    exact = S * K * 4 if T <= 16 else 0
    return {
        "moe_grouped_gate_up": distinct * gu + T * K * 2 + S * F * 2,
        "moe_grouped_down": distinct * dn + S * F * 2 + S * K * 2,      # y in fp16
        "moe_decode_gate_up": distinct * gu + T * K * 4 + S * F * 4 + exact,
        # with the certified selection in its prologue: also reads S and B
        "moe_decode_gate_up_sel": distinct * gu + T * K * 4 + S * F * 4 + T * E * (8 + 4) + exact,
        "moe_decode_down": distinct * dn + S * F * 4 + T * K * 4,
        # on the grouped path (T > 16 by default) the router launch also writes x in fp16
        "router_logits": W.router_bytes(spec) + T * K * 4 + T * E * 4 + (T * K * 2 if T > 16 else 0),
        # certified router: the sums read the router and x, write S, B and the logits;
        # the selection reads S and B
        "router_sums": W.router_bytes(spec) + T * K * 4 + T * E * (8 + 4 + 4),
        "router_select": T * E * (8 + 4),
    }.get(name)


def load_traffic(args):
    tpath = Path(args.traffic) if args.traffic else ROOT / "profiles" / "hbm_traffic.json"
    return json.loads(tpath.read_text()) if tpath.exists() else None


def held(step):
    """step(i) preceded by a hold of the stream long enough for the host to
    enqueue the step before the GPU reaches it, for the passes that bracket
    kernels with events: where the host enqueues more slowly than the GPU runs
    (T = 1), an event pair around a kernel would otherwise also span the
    host's launch of that kernel.  The hold is sized from the host's enqueue
    time of one step, measured with the stream held."""
    from qw3_amd._native import hip
    hip().ds3_hip_synchronize()
    hip().ds3_hip_begin_batch()
    hip().ds3_hip_hold_stream(20000.0)
    t0 = time.perf_counter()
    step(0)
    host_us = (time.perf_counter() - t0) * 1e6
    hip().ds3_hip_end_batch()
    hold_us = min(20000.0, 2.0 * host_us + 50.0)

    def run(i):
        hip().ds3_hip_hold_stream(hold_us)
        step(i)
    return run


BRK_STEPS = 20                 # steps of the per-kernel breakdown pass


def time_steps(step, steps, warmup, spec, T, n_used, first, per_kernel=True, graph_of=0):
    """`first()` runs one step and returns the routed indices [T][n_used];
    then `warmup` plain untimed steps back to back (the GPU reaches its
    sustained clocks and the layers' address translations are warm: the first
    few milliseconds of a burst run ~10 % slower), the timed steps with no
    per-kernel events, BRK_STEPS steps with every kernel bracketed by events
    (the breakdown, which names the dominant kernel), and the timed steps
    again with only the dominant kernel bracketed (its mean duration for the
    roofline).  The two event passes follow the timed region, so they see the
    same sustained state.  With graph_of = G > 0 the warmup and timed steps
    are replays of one HIP graph of steps 0 .. G-1 (steps a multiple of G), as
    a decode loop replays its captured calls.  Returns (wall_ms, gpu_ms,
    stats, breakdown, counts)."""
    from qw3_amd import ds3
    from qw3_amd._native import hip
    E = spec.n_expert
    idx = first()
    hip().ds3_hip_synchronize()
    counts = np.bincount(idx.reshape(-1), minlength=E)
    graph = None
    if graph_of:
        assert steps % graph_of == 0
        graph = ds3.Graph()
        with graph:
            for i in range(graph_of):
                step(i)
    # warmup: plain steps (graph replays), enqueued back to back and untimed
    hip().ds3_hip_begin_batch()
    if graph is not None:
        for _ in range(max(1, warmup // graph_of)):
            graph.launch()
    else:
        for i in range(warmup):
            step(i)
    hip().ds3_hip_end_batch()
    # timed region: synchronise, K steps enqueued back to back, synchronise;
    # no per-kernel events in it (at T = 1 an event pair costs a third of a step)
    hip().ds3_hip_synchronize()
    hip().ds3_hip_begin_batch()
    t0 = time.perf_counter()
    hip().ds3_hip_timer_start()
    if graph is not None:
        for _ in range(steps // graph_of):
            graph.launch()
    else:
        for i in range(steps):
            step(i)
    gpu_ms = hip().ds3_hip_timer_stop_ms()
    hip().ds3_hip_end_batch()
    wall_ms = (time.perf_counter() - t0) * 1e3
    if graph is not None:
        graph.close()
    brk, stats = {}, {}
    if per_kernel:
        hstep = held(step)
        # breakdown: every kernel bracketed by events on the library's stream
        hip().ds3_hip_kernel_timing_only(None)
        hip().ds3_hip_kernel_timing_reset()
        hip().ds3_hip_kernel_timing(1)
        hip().ds3_hip_begin_batch()
        for i in range(BRK_STEPS):
            hstep(i)
        hip().ds3_hip_end_batch()
        hip().ds3_hip_kernel_timing(0)
        brk = ds3.kernel_stats()
        dominant = max((k for k in brk if kernel_bytes(k, spec, T, counts, n_used) is not None),
                       key=lambda k: brk[k][1])
        # the timed steps again with only the dominant kernel bracketed
        hip().ds3_hip_kernel_timing_reset()
        hip().ds3_hip_kernel_timing_only(dominant.encode())
        hip().ds3_hip_kernel_timing(1)
        hip().ds3_hip_begin_batch()
        for i in range(steps):
            hstep(i)
        hip().ds3_hip_end_batch()
        hip().ds3_hip_kernel_timing(0)
        hip().ds3_hip_kernel_timing_only(None)
        stats = ds3.kernel_stats()
    return wall_ms, gpu_ms, stats, brk, counts


def layer_steps(T, layers, xs, spec, n_used=8, noalloc=False, zero=True):
    """(step, first) for one layer call per step on T tokens, layers cycled.
    zero: the step first zeroes the output, as the engine's gathered prefill
    does (reference src/ds3_engine.c:902); otherwise every call accumulates
    into it, as a decode step adds the layer's output to the residual stream."""
    from qw3_amd import ds3
    E, K = spec.n_expert, spec.n_embd
    out = ds3.Buffer.alloc(T * K * 4)
    idx = ds3.Buffer.alloc(T * n_used * 4)

    def step(i, want_idx=False):
        d = layers[i % len(layers)]
        if zero:
            out.zero()
        ds3.moe_ffn_batch(xs[i % len(xs)], d.router, spec.router_type, d.experts, out, T, E, n_used,
                          indices=idx if want_idx else None)

    def first():
        step(0, True)
        return idx.read(np.int32, (T, n_used))

    return step, first


def roofline(stats, spec, T, counts, n_used, traffic):
    """traffic: {kernel: HBM bytes per launch} measured at T = 512, and at
    T = 1 under "T1/<kernel>" (T = 2048 under "T2048/"); the all-Q8_0 layer's
    under "Q8_0/T<T>/"."""
    name = next(iter(stats))                  # the one kernel timed in the second pass
    n, ms = stats[name]
    avg_s = ms / n / 1e3
    b = kernel_bytes(name, spec, T, counts, n_used)
    achieved = b / avg_s / 1e9
    r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": name,
         "kernel_avg_us": round(avg_s * 1e6, 2), "alg_bytes_per_launch": b}
    if spec.gate_type == 12:
        key = {1: "T1/", 512: "", 2048: "T2048/"}.get(T)
    elif spec.gate_type == 8:
        key = f"Q8_0/T{T}/"
    else:
        key = None
    if traffic and key is not None and key + name in traffic:
        r["traffic"] = traffic[key + name]
    return r


def log_breakdown(brk, stats):
    log(f"[bench]   breakdown pass ({BRK_STEPS} steps), every kernel bracketed by events:")
    for k, (n, ms) in sorted(brk.items(), key=lambda kv: -kv[1][1]):
        log(f"[bench]     {k:24s} {n:5d} launches  avg {ms / n * 1e3:8.2f} us")
    for k, (n, ms) in stats.items():
        log(f"[bench]   timed region, {k} alone: {n} launches avg {ms / n * 1e3:.2f} us")


# ---------------------------------------------------------------------------
# CPU baseline: the reference's ds3_ref_moe_ffn per token (oracle port where
# the reference was not built), FP32-dequantised weights resident
# ---------------------------------------------------------------------------

def host_cores():
    return {"host_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}


class CpuLayer:
    """A host layer dequantised to FP32 the way the reference's tests feed it
    (ds3_ref_dequantize_tensor once per layer, untimed)."""

    def __init__(self, host):
        sys.path.insert(0, str(ROOT / "tests"))
        import _oracle as O
        self.O = O
        spec = host.spec
        self.spec = spec
        E, K, F = spec.n_expert, spec.n_embd, spec.n_ff
        self.kind = "reference" if O.ref() is not None else "port"
        deq = O.ref_dequantize if self.kind == "reference" else O.dequantize
        self.wr = deq(spec.router_type, host.router, E * K) if spec.router_type != 0 else host.router.view(np.float32)
        self.wg = deq(spec.gate_type, host.gate, E * F * K)
        self.wu = deq(spec.up_type, host.up, E * F * K)
        self.wd = deq(spec.down_type, host.down, E * K * F)
        self.fn = O.ref().ds3_ref_moe_ffn if self.kind == "reference" else O.orc().orc_moe_ffn

    def ffn(self, x, out, n_used, scratch):
        O, s = self.O, self.spec
        lg, sc, ix = scratch
        self.fn(O.ptr(x), O.ptr(self.wr), O.ptr(self.wg), O.ptr(self.wu), O.ptr(self.wd), None, None, None,
                O.ptr(out), O.ptr(lg), O.ptr(sc), O.ptr(ix), s.n_embd, s.n_expert, n_used, s.n_ff, 0, True)


def _scratch(spec, n_used):
    return np.empty(spec.n_expert, np.float32), np.empty(n_used, np.float32), np.empty(n_used, np.int32)


def cpu_tokens(cl, x, n_used, threads):
    """Tokens/s of ds3_ref_moe_ffn over the rows of x on `threads` host
    threads (ctypes releases the GIL during each call)."""
    import concurrent.futures as cf
    n = x.shape[0]
    out = np.empty_like(x)

    def work(r):
        s = _scratch(cl.spec, n_used)
        for t in r:
            cl.ffn(x[t], out[t], n_used, s)

    t0 = time.perf_counter()
    if threads == 1:
        work(range(n))
    else:
        with cf.ThreadPoolExecutor(threads) as ex:
            list(ex.map(work, [range(i, n, threads) for i in range(threads)]))
    return n / (time.perf_counter() - t0), time.perf_counter() - t0


def pinned_one_core(fn):
    """Run fn() on this thread pinned to one host core; returns (result, core)."""
    prev = os.sched_getaffinity(0)
    core = min(prev)
    os.sched_setaffinity(0, {core})
    try:
        return fn(), core
    finally:
        os.sched_setaffinity(0, prev)


def cpu_baseline(host, x, n_used, n_threaded, n_single, what):
    """Multi-thread figure (the main object) with the 1-core pinned figure beside it."""
    t0 = time.perf_counter()
    cl = CpuLayer(host)
    log(f"[bench] cpu baseline ({what}): dequantised layer in {time.perf_counter() - t0:.1f}s ({cl.kind})")
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    xt = np.ascontiguousarray(x[:n_threaded])
    v, dt = cpu_tokens(cl, xt, n_used, threads)
    xs = np.ascontiguousarray(x[:n_single])
    (v1, dt1), core = pinned_one_core(lambda: cpu_tokens(cl, xs, n_used, 1))
    log(f"[bench] cpu baseline ({what}): {v:.1f} tok/s on {threads} threads, {v1:.2f} tok/s on 1 core")
    return {"value": round(v, 2), "unit": "tokens/s", "cores": threads, "kind": cl.kind,
            "sample": f"{xt.shape[0]} tokens of {what}, one layer, FP32-dequantised weights resident, "
                      f"ds3_ref_moe_ffn per token on {threads} threads ({dt:.1f}s wall)",
            "one_core": {"value": round(v1, 3), "unit": "tokens/s", "cores": 1, "pinned_cpu": core,
                         "sample": f"{xs.shape[0]} tokens, one thread pinned to cpu {core} ({dt1:.1f}s wall)"},
            **host_cores()}


# ---------------------------------------------------------------------------
# Legs
# ---------------------------------------------------------------------------

def make_layers(spec, n, what):
    from qw3_amd import workload as W
    t0 = time.perf_counter()
    hosts, layers = [], []
    for l in range(n):
        h = W.make_layer(spec, seed=1234, layer=l)
        layers.append(h.to_device(readonly=True))       # as the engine imports mmap'd GGUF weights
        if l == 0:
            hosts.append(h)
    log(f"[bench] {what}: {n} layers generated and resident in {time.perf_counter() - t0:.1f}s")
    return hosts[0], layers


def leg_layer(args, config, T, steps, warmup, spec, layers, xs, traffic, n_used=8, what="", graph_of=0,
              zero=True):
    """One layer call per step on T tokens: figures, dominant-kernel roofline."""
    from qw3_amd import workload as W
    step, first = layer_steps(T, layers, xs, spec, n_used, zero=zero)
    wall_ms, gpu_ms, stats, brk, counts = time_steps(step, steps, warmup, spec, T, n_used, first,
                                                     graph_of=graph_of)
    ms = wall_ms / steps
    log(f"[bench] {what} T={T}: {ms * 1e3:.1f} us/step wall, {gpu_ms / steps * 1e3:.1f} us/step events"
        + (f", steps replayed as HIP graphs of {graph_of}" if graph_of else ""))
    log_breakdown(brk, stats)
    distinct = int((counts > 0).sum())
    b = W.algorithmic_bytes(spec, T, distinct)
    flops = W.algorithmic_flops(spec, T, n_used)
    return {
        "value": round(T / (ms / 1e3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "steps": steps,
        "warmup": warmup, "tokens": T, "alg_bytes_per_step": b,
        "hbm_frac_step": round(b / (ms / 1e3) / (HBM_PEAK_GBS * 1e9), 4),
        "mfma_util": round(flops / (ms / 1e3) / (FP16_PEAK_TFLOPS * 1e12), 4),
        "roofline": roofline(stats, spec, T, counts, n_used, traffic),
        "kernels_us": {k: round(v[1] / v[0] * 1e3, 2) for k, v in brk.items()},
        "distinct_experts": distinct,
        "expert_histogram": {"max_tokens": int(counts.max()), "min_tokens": int(counts.min()),
                             "experts_0": int((counts == 0).sum()),
                             "experts_1_2": int(((counts >= 1) & (counts <= 2)).sum()),
                             "top_share": round(float(counts.max()) / float(counts.sum()), 4)},
    }


def leg_c3(args, traffic):
    """T = 2048 with Zipf-skewed routing; MFMA-bound (AI ~365)."""
    from qw3_amd import ds3
    from qw3_amd import workload as W
    spec = W.config_spec(3)
    host, layers = make_layers(spec, 4, "c3")
    xh = [W.make_inputs(3, 2048, seed=99, step=s) for s in range(2)]
    xs = [ds3.Buffer.from_array(x) for x in xh]
    r = leg_layer(args, 3, 2048, 100, 20, spec, layers, xs, traffic, what="c3")
    flops = W.algorithmic_flops(spec, 2048)
    r["mfma_roofline"] = {"bound": "mfma", "achieved": round(flops / (r["ms_per_step"] / 1e3) / 1e12, 1),
                          "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": r["mfma_util"],
                          "alg_flops_per_step": flops}
    r["workload"] = ("configs[2]: one Qwen3-30B-A3B MoE-FFN layer, T=2048, router U(-a,a) plus a Zipf(s=1.2) "
                     "per-expert logit bias through x[:,2047]=1; Q4_K gate/up + Q6_K down, F32 router")
    if not args.no_cpu:
        r["cpu_baseline"] = cpu_baseline(host, xh[0], 8, 512, 24, "the T=2048 Zipf batch")
    return r


def leg_c5(args, traffic):
    """all-Q8_0 layer; every T on the GEMV path and on the grouped
    path, the step's HBM roofline fraction each, and the crossover."""
    from qw3_amd import ds3
    from qw3_amd import workload as W
    from qw3_amd._native import hip
    spec = W.config_spec(5)
    host, layers = make_layers(spec, 4, "c5")
    default_min = hip().ds3_hip_set_prefill_min_tokens(0)
    hip().ds3_hip_set_prefill_min_tokens(default_min)
    sweep = {}
    for T in C5_TOKENS:
        xh = [W.make_inputs(5, T, seed=99, step=s) for s in range(4)]
        xs = [ds3.Buffer.from_array(x) for x in xh]
        row = {}
        for path, mn in (("gemv", 1 << 30), ("grouped", 1)):
            ds3.set_prefill_min_tokens(mn)
            steps = 200 if T <= 64 else 50
            step, first = layer_steps(T, layers, xs, spec)
            wall_ms, _, _, _, counts = time_steps(step, steps, steps // 5, spec, T, 8, first, per_kernel=False)
            ms = wall_ms / steps
            b = W.algorithmic_bytes(spec, T, int((counts > 0).sum()))
            row[path] = {"ms_per_step": round(ms, 5), "tokens_per_s": round(T / (ms / 1e3), 1),
                         "hbm_frac_step": round(b / (ms / 1e3) / (HBM_PEAK_GBS * 1e9), 4),
                         "alg_bytes_per_step": b}
        ds3.set_prefill_min_tokens(default_min)
        row["faster"] = min(("gemv", "grouped"), key=lambda p: row[p]["ms_per_step"])
        row["default_path"] = "grouped" if T >= default_min else "gemv"
        log(f"[bench] c5 T={T}: gemv {row['gemv']['ms_per_step'] * 1e3:.1f} us, "
            f"grouped {row['grouped']['ms_per_step'] * 1e3:.1f} us (default: {row['default_path']})")
        sweep[str(T)] = row
    # dominant-kernel roofline at the headline-sized T of the sweep, default path
    T = 256
    xs = [ds3.Buffer.from_array(W.make_inputs(5, T, seed=99, step=s)) for s in range(4)]
    dom = leg_layer(args, 5, T, 100, 20, spec, layers, xs, traffic, what="c5")
    faster = [int(t) for t, r in sweep.items() if r["faster"] == "grouped"]
    slower = [int(t) for t, r in sweep.items() if r["faster"] == "gemv"]
    r = {"sweep": sweep, "prefill_min_tokens": default_min,
         "crossover": {"gemv_faster_at": slower, "grouped_faster_at": faster},
         "T256": dom,
         "workload": "configs[4]: one layer with every expert matrix and the router in Q8_0, x ~ N(0,1)"}
    if not args.no_cpu:
        r["cpu_baseline"] = cpu_baseline(host, W.make_inputs(5, 256, seed=99), 8, 256, 24, "the Q8_0 layer, T=256")
    return r


def leg_dense(args, traffic):
    """The engine's dense quantised products beside the MoE (reference
    src/ds3_engine.c:181-271): the output head (2048 -> 151,936 logits, one
    token: vec_matmul, HBM-bound) in Q6_K and Q8_0, and a prefill projection
    (M = 512 rows, 2048 -> 4096, Q4_K: matmul_quantized_batch) on its fp16
    MFMA path and on its fp32 path.  Two weight copies alternate per call so
    the head's 255-330 MB cannot stay in the 256 MB Infinity Cache.  The
    head's measured traffic per launch is under "head/<type>/gemv1"."""
    from qw3_amd import ds3
    from qw3_amd import workload as W
    from qw3_amd._native import hip
    K, NH = 2048, 151936
    out = {"workload": "output head 2048 -> 151,936 (one token) in Q6_K and Q8_0; prefill projection "
                       "512 x 2048 -> 4096 in Q4_K; weights N(0, 0.02) quantised, x ~ N(0, 1)"}
    rng = np.random.default_rng(5)
    x = ds3.Buffer.from_array(rng.standard_normal(K).astype(np.float32))
    y = ds3.Buffer.alloc(NH * 4)

    def timed(name, call, n):
        hip().ds3_hip_kernel_timing_reset()
        hip().ds3_hip_kernel_timing_only(name.encode())
        hip().ds3_hip_kernel_timing(1)
        hip().ds3_hip_begin_batch()
        t0 = time.perf_counter()
        for i in range(n):
            call(i)
        hip().ds3_hip_end_batch()
        wall = (time.perf_counter() - t0) / n
        hip().ds3_hip_kernel_timing(0)
        hip().ds3_hip_kernel_timing_only(None)
        cnt, ms = ds3.kernel_stats()[name]
        return ms / cnt / 1e3, wall

    head = {}
    for t in (ds3.TYPE_Q6_K, ds3.TYPE_Q8_0):
        raw = W.quant_matrix(t, W.NORMAL, 7, t, NH, K, 0.0, 0.02)
        ws = [ds3.Buffer.from_array(raw) for _ in range(2)]
        rs = ds3.row_bytes(t, K)
        call = lambda i: hip().ds3_hip_vec_matmul_quantized(x, ws[i % 2], y, K, NH, rs, t)
        for i in range(4):
            call(i)
        k_s, wall = timed("gemv1", call, 40)
        b = NH * rs + K * 4 + NH * 4
        head[ds3.TYPE_NAMES[t]] = {
            "us_per_call": round(k_s * 1e6, 2), "wall_us_per_call": round(wall * 1e6, 2), "alg_bytes": b,
            "roofline": {"bound": "hbm", "achieved": round(b / k_s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(b / k_s / 1e9 / HBM_PEAK_GBS, 4),
                         "traffic": (traffic or {}).get(f"head/{ds3.TYPE_NAMES[t]}/gemv1"), "kernel": "gemv1"}}
        log(f"[bench] dense: head {ds3.TYPE_NAMES[t]} {k_s * 1e6:.1f} us ({b / k_s / 1e12:.2f} TB/s)")
        if t == ds3.TYPE_Q6_K and not args.no_cpu:
            sys.path.insert(0, str(ROOT / "tests"))
            import _oracle as O
            Wf = (O.ref_dequantize if O.ref() is not None else O.dequantize)(t, raw, NH * K)
            xh = np.ascontiguousarray(rng.standard_normal(K).astype(np.float32))
            yh = np.empty(NH, np.float32)
            fn = O.ref().ds3_ref_vec_matmul if O.ref() is not None else O.orc().orc_vec_matmul

            def one():
                t1 = time.perf_counter()
                for _ in range(3):
                    fn(O.ptr(xh), O.ptr(Wf), O.ptr(yh), K, NH)
                return (time.perf_counter() - t1) / 3
            dt, core = pinned_one_core(one)
            head["Q6_K"]["cpu_baseline"] = {
                "value": round(1.0 / dt, 3), "unit": "calls/s", "cores": 1,
                "kind": "reference" if O.ref() is not None else "port", "pinned_cpu": core,
                "sample": f"3 calls of ds3_ref_vec_matmul 2048 -> 151,936 on FP32-dequantised weights, one pinned "
                          f"thread ({dt * 1e3:.0f} ms per call)", **host_cores()}
            del Wf
        del ws
    out["head"] = head
    M, N = 512, 4096
    t = ds3.TYPE_Q4_K
    raw = W.quant_matrix(t, W.NORMAL, 8, t, N, K, 0.0, 0.02)
    wb = ds3.Buffer.from_array(raw)
    A = ds3.Buffer.from_array(rng.standard_normal((M, K)).astype(np.float32))
    C = ds3.Buffer.alloc(M * N * 4)
    rs = ds3.row_bytes(t, K)
    flops = 2 * M * N * K
    proj = {"rows": M, "N": N, "K": K, "type": "Q4_K", "alg_flops": flops}
    for name, min_rows in (("dense_mfma", 1), ("gemv", 1 << 30)):
        prev = hip().ds3_hip_set_dense_mfma_min_rows(min_rows)
        call = lambda i: hip().ds3_hip_matmul_quantized_batch(A, wb, C, M, N, K, rs, 0, t)
        call(0)
        k_s, wall = timed(name, call, 10)
        hip().ds3_hip_set_dense_mfma_min_rows(prev)
        key = "mfma_fp16" if name == "dense_mfma" else "fp32"
        proj[key] = {"us_per_call": round(k_s * 1e6, 2), "wall_us_per_call": round(wall * 1e6, 2),
                     "tflops": round(flops / k_s / 1e12, 2)}
        log(f"[bench] dense: projection {M}x{K}->{N} Q4_K {key}: {k_s * 1e6:.1f} us ({flops / k_s / 1e12:.1f} TFLOP/s)")
    proj["mfma_roofline"] = {"bound": "mfma", "achieved": proj["mfma_fp16"]["tflops"], "peak": FP16_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(proj["mfma_fp16"]["tflops"] / FP16_PEAK_TFLOPS, 4)}
    out["projection"] = proj
    return out


def leg_stack(args, traffic, n_used=8):
    """one token per step through a resident stack of
    --stack-layers MoE layers, h <- h + MoE_l(h) in place (the call
    accumulates into its own input), as the engine runs decode; replayed as
    one HIP graph per token unless --no-graph.  With --stack-block each layer
    is the engine's whole FFN block, h <- h + MoE_l(rms_norm(h) * g_l)."""
    from qw3_amd import ds3
    from qw3_amd import workload as W
    from qw3_amd._native import hip
    spec = W.config_spec(4)
    L, K, E = args.stack_layers, spec.n_embd, spec.n_expert
    t0 = time.perf_counter()
    hosts, layers = [], []
    for l in range(L):
        h = W.make_layer(spec, seed=1234, layer=l)
        layers.append(h.to_device(readonly=True))       # as the engine imports mmap'd GGUF weights
        if l < 2 and not args.no_cpu:
            hosts.append(h)
    log(f"[bench] c4: {L} layers generated and resident in {time.perf_counter() - t0:.1f}s "
        f"({L * (W.expert_bytes(spec) * E + W.router_bytes(spec)) / 2**30:.2f} GiB)")
    hs_host = [W.make_inputs(4, 1, seed=99, step=s) for s in range(8)]
    hs = [ds3.Buffer.from_array(x) for x in hs_host]
    h = ds3.Buffer.alloc(K * 4)
    idx = ds3.Buffer.alloc(n_used * 4)
    gains = [ds3.Buffer.from_array((1.0 + W.fill(W.NORMAL, 700 + l, 1, K, 0.0, 0.02)).astype(np.float32))
             for l in range(L)] if args.stack_block else None

    def layer_call(l, d, ix=None):
        if gains is not None:
            ds3.moe_block(h, gains[l], 1e-6, d.router, spec.router_type, d.experts, 1, E, n_used, indices=ix)
        else:
            ds3.moe_ffn_batch(h, d.router, spec.router_type, d.experts, h, 1, E, n_used, indices=ix)

    def token(i):
        hip().ds3_hip_buffer_copy_f32(hs[i % len(hs)], h, K * 4)     # a fresh hidden state, on the device
        for l, d in enumerate(layers):
            layer_call(l, d)

    def first():
        hip().ds3_hip_buffer_copy_f32(hs[0], h, K * 4)
        for l, d in enumerate(layers):
            layer_call(l, d, idx if l == 0 else None)
        return idx.read(np.int32, (n_used,))

    graph = None
    step = token
    if not args.no_graph:
        token(0)                               # sizes the workspace before the capture
        graph = ds3.Graph()
        with graph:
            for l, d in enumerate(layers):
                layer_call(l, d)

        def step(i):
            hip().ds3_hip_buffer_copy_f32(hs[i % len(hs)], h, K * 4)
            graph.launch()

    # graph replays record no per-kernel events: the breakdown and the
    # dominant kernel's events come from eager tokens after the timed region
    # (`token`, the function the graph captured)
    steps = args.stack_steps
    idx0 = first()
    counts = np.bincount(idx0, minlength=E)
    htoken = held(token)
    hip().ds3_hip_begin_batch()
    for i in range(args.warmup):
        step(i)
    hip().ds3_hip_end_batch()
    hip().ds3_hip_synchronize()
    hip().ds3_hip_begin_batch()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    hip().ds3_hip_end_batch()
    wall_ms = (time.perf_counter() - t0) * 1e3
    # the event passes after the timed region, in the same sustained state
    hip().ds3_hip_kernel_timing_only(None)
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing(1)
    hip().ds3_hip_begin_batch()
    for i in range(2):
        htoken(i)
    hip().ds3_hip_end_batch()
    hip().ds3_hip_kernel_timing(0)
    brk = ds3.kernel_stats()
    dominant = max((k for k in brk if kernel_bytes(k, spec, 1, counts, n_used) is not None), key=lambda k: brk[k][1])
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing_only(dominant.encode())
    hip().ds3_hip_kernel_timing(1)
    hip().ds3_hip_begin_batch()
    for i in range(steps):
        htoken(i)
    hip().ds3_hip_end_batch()
    hip().ds3_hip_kernel_timing(0)
    hip().ds3_hip_kernel_timing_only(None)
    stats = ds3.kernel_stats()
    if graph:
        graph.close()
    ms = wall_ms / steps
    log(f"[bench] c4: {ms * 1e3:.1f} us/token through {L} layers ({ms * 1e3 / L:.2f} us/layer)"
        + (", layers replayed as one HIP graph" if graph else ""))
    log_breakdown(brk, stats)
    b = L * W.algorithmic_bytes(spec, 1, n_used)
    r = {
        "value": round(1 / (ms / 1e3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "steps": steps,
        "warmup": args.warmup, "layers": L, "alg_bytes_per_step": b, "hbm_frac_step": round(b / (ms / 1e3) / (HBM_PEAK_GBS * 1e9), 4),
        "us_per_layer": round(ms * 1e3 / L, 3), "graph": graph is not None, "stack_block": bool(args.stack_block),
        "roofline": roofline(stats, spec, 1, counts, n_used, traffic),
        "workload": f"configs[3]: decode, one token per step through {L} resident Qwen3-30B-A3B MoE-FFN layers "
                    f"({L * (W.expert_bytes(spec) * E + W.router_bytes(spec)) / 2**30:.2f} GiB), "
                    + ("h <- h + MoE_l(rms_norm(h) * g_l)" if args.stack_block else "h <- h + MoE_l(h)")
                    + "; Q4_K gate/up + Q6_K down, F32 router"
                    + ("" if args.no_graph else "; the token's layers replayed as one HIP graph"),
    }
    if not args.no_cpu and not args.stack_block:
        r["cpu_baseline"] = cpu_stack(hosts, hs_host, L, n_used)
    return r


def cpu_stack(hosts, hs_host, L, n_used):
    """Config 4 on the host: token streams through a stated subset of resident
    layers (FP32 copies of 48 layers would need ~116 GB), each token
    h <- h + ds3_ref_moe_ffn_l(h) as the reference's engine does per layer;
    tokens/s through L layers = the subset's rate x subset / L."""
    import concurrent.futures as cf
    cls = [CpuLayer(hh) for hh in hosts]
    sub = len(cls)
    K = cls[0].spec.n_embd
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    n_tok = 4 * threads

    def run(tokens):
        s = _scratch(cls[0].spec, n_used)
        y = np.empty(K, np.float32)
        for t in tokens:
            h = hs_host[t % len(hs_host)].reshape(-1).copy()
            for cl in cls:
                y[:] = 0.0
                cl.ffn(h, y, n_used, s)
                h += y
        return len(tokens)

    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(threads) as ex:
        list(ex.map(run, [range(i, n_tok, threads) for i in range(threads)]))
    dt = time.perf_counter() - t0
    v = n_tok / dt * sub / L
    n1 = 6

    def one():
        t1 = time.perf_counter()
        run(range(n1))
        return time.perf_counter() - t1

    dt1, core = pinned_one_core(one)
    v1 = n1 / dt1 * sub / L
    log(f"[bench] cpu baseline (c4): {v:.2f} tok/s through {L} layers on {threads} threads, {v1:.3f} on 1 core")
    return {"value": round(v, 3), "unit": "tokens/s", "cores": threads, "kind": cls[0].kind,
            "sample": f"{n_tok} token streams through {sub} resident layers (h <- h + ds3_ref_moe_ffn(h)) on "
                      f"{threads} threads ({dt:.1f}s wall), extrapolated to {L} layers (x {sub}/{L})",
            "one_core": {"value": round(v1, 4), "unit": "tokens/s", "cores": 1, "pinned_cpu": core,
                         "sample": f"{n1} tokens through {sub} layers on one pinned thread ({dt1:.1f}s), "
                                   f"extrapolated to {L} layers"},
            **host_cores()}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "see DESIGN.md for how the MoE FFN would shard across GPUs.", file=sys.stderr)
        sys.exit(2)
    from qw3_amd import ds3
    from qw3_amd import workload as W
    ds3.init()
    info = ds3.device_info()
    log(f"[bench] device {info['arch']} CUs={info['n_cu']}")
    traffic = load_traffic(args)
    if args.copy_mib:
        from qw3_amd._native import hip
        n = args.copy_mib << 20
        a, b = ds3.Buffer.alloc(n), ds3.Buffer.alloc(n)
        for _ in range(3):
            if hip().ds3_hip_buffer_copy_f32(a, b, n) != 0:
                raise RuntimeError("buffer_copy_f32 failed")
        hip().ds3_hip_synchronize()
        log(f"[bench] copy calibration: 3 x {args.copy_mib} MiB device copy")
        a.close()
        b.close()
    if args.config == 4:
        r = leg_stack(args, traffic)
        line = {"metric": f"decode tokens/s through a {args.stack_layers}-layer resident MoE-FFN stack "
                          f"(configs[3]); HBM GB/s vs peak",
                "value": r["value"], "unit": "tokens/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
                "ms_per_step": r["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                "dtype": "f16", "data": "synthetic (seeded generator; expert weights N(0,0.02) quantised by this "
                                        "project's GGUF quantisers)",
                "config": {"workload": r["workload"], "tokens": 1, "layers": args.stack_layers},
                "roofline": r["roofline"], **{k: v for k, v in r.items() if k not in ("roofline", "workload")}}
        print(json.dumps(line), flush=True)
        return
    if args.config in (3, 5) and args.tokens is None:
        r = leg_c3(args, traffic) if args.config == 3 else leg_c5(args, traffic)
        print(json.dumps({"metric": f"configs[{args.config - 1}]", "n_gpus": 1, **r}), flush=True)
        return

    config = args.config or 2
    spec = W.config_spec(config)
    T, n_used = args.tokens or 512, W.N_USED
    host, layers = make_layers(spec, args.layers, f"c{config}")
    xs_host = [W.make_inputs(config, T, seed=99, step=s) for s in range(4)]
    xs = [ds3.Buffer.from_array(x) for x in xs_host]
    main_leg = leg_layer(args, config, T, args.steps, args.warmup, spec, layers, xs, traffic, what=f"c{config}")
    line = {
        "metric": "MoE-FFN tokens/s at T=512 (T=1 under t1; configs 3-5 under c3, c4, c5); "
                  "HBM GB/s and MFMA util vs peak",
        "value": main_leg["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_leg["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded generator; expert weights N(0,0.02) quantised by this project's GGUF quantisers)",
        "config": {"workload": f"configs[{config - 1}]: one Qwen3-30B-A3B MoE-FFN layer, T={T} gathered prefill, "
                               f"{W.N_EXPERT} experts top-{n_used}, "
                               f"{ds3.TYPE_NAMES[spec.gate_type]} gate/up + {ds3.TYPE_NAMES[spec.down_type]} down, "
                               f"{ds3.TYPE_NAMES[spec.router_type]} router",
                   "tokens": T, "n_embd": spec.n_embd, "n_ff": spec.n_ff, "layers_cycled": args.layers,
                   "distinct_experts_step0": main_leg["distinct_experts"]},
        "roofline": main_leg["roofline"],
        "mfma_util": main_leg["mfma_util"],
        "alg_bytes_per_step": main_leg["alg_bytes_per_step"],
        "hbm_frac_step": main_leg["hbm_frac_step"],
        "kernels_us": main_leg["kernels_us"],
    }
    if not args.no_t1 and config == 2:
        spec1 = W.config_spec(1)
        layers1 = [W.make_layer(spec1, seed=1234, layer=l).to_device(readonly=True) for l in range(args.layers)]
        x1h = [W.make_inputs(1, 1, seed=98, step=s) for s in range(16)]
        x1 = [ds3.Buffer.from_array(x) for x in x1h]
        # decode: the timed steps replay a HIP graph of 16 steps (every layer
        # and input pair once), as a decode loop replays its captured calls
        # (--no-graph: each step enqueued from Python)
        g = 0 if args.no_graph else 16
        t1_steps = args.t1_steps if not g else max(g, args.t1_steps // g * g)
        t1 = leg_layer(args, 1, 1, t1_steps, args.warmup, spec1, layers1, x1, traffic, what="t1", graph_of=g,
                       zero=args.t1_zero)
        t1["graph"] = bool(g)
        t1["output_zeroed_per_step"] = bool(args.t1_zero)
        for k in ("mfma_util", "expert_histogram", "tokens"):
            t1.pop(k, None)
        if not args.no_cpu:
            host1 = W.make_layer(spec1, seed=1234, layer=0)
            cl = CpuLayer(host1)
            xs1 = np.concatenate(x1h)
            (v1, dt1), core = pinned_one_core(lambda: cpu_tokens(cl, xs1, n_used, 1))
            t1["cpu_baseline"] = {"value": round(v1, 3), "unit": "tokens/s", "cores": 1, "kind": cl.kind,
                                  "pinned_cpu": core,
                                  "sample": f"{xs1.shape[0]} single-token calls of ds3_ref_moe_ffn on one pinned "
                                            f"thread ({dt1:.1f}s wall): one token cannot be split over threads",
                                  **host_cores()}
        line["t1"] = t1
        del layers1
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(host, xs_host[0], n_used, min(args.cpu_tokens, T), min(48, T),
                                            f"the T={T} batch")
    if args.config == 0:
        skip = set(s for s in args.skip.split(",") if s)
        del layers
        if "c3" not in skip:
            line["c3"] = leg_c3(args, traffic)
        if "c5" not in skip:
            line["c5"] = leg_c5(args, traffic)
        if "c4" not in skip:
            line["c4"] = leg_stack(args, traffic)
        if "dense" not in skip:
            line["dense"] = leg_dense(args, traffic)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
