"""MoE-FFN throughput on one MI355X (benchmark contract: one JSON line on stdout).

Workload: one Qwen3-30B-A3B MoE-FFN layer call on
T = 512 tokens -- router, softmax/top-8, bucketing, grouped Q4_K gate/up and
Q6_K down products, SwiGLU and the weighted combine -- through the C ABI
(ds3_hip_moe_ffn_batch).  A step is one layer call on one batch; the engine's
output zeroing (reference src/ds3_engine.c:902) is part of the step.  Layers
are cycled from `--layers` distinct resident copies so weights cannot stay in
the 256 MB Infinity Cache between steps.  The line also carries the T = 1
decode figures (configs[0] shape) under "t1".

roofline: the dominant kernel's algorithmic bytes per launch / its mean
duration, timed with HIP events on the library stream over a second pass of
the same K steps (the timed region itself carries no per-kernel events).
cpu_baseline: the reference's own ds3_ref_moe_ffn (compiled from its sources
into oracle/_ref) on the host cores, FP32-dequantised weights resident, on a
bounded sample of the same workload.
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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--tokens", type=int, default=512)
    p.add_argument("--layers", type=int, default=8, help="distinct resident layers cycled per step")
    p.add_argument("--config", type=int, default=2, choices=(2, 3, 4, 5),
                   help="2, 3, 5: one layer on --tokens tokens (+ T=1 under t1); 4: the decode stack")
    p.add_argument("--stack-layers", type=int, default=48, help="config 4: resident layers per decode step")
    p.add_argument("--no-graph", action="store_true",
                   help="config 4: enqueue every layer eagerly instead of replaying the token's layers as one HIP graph")
    p.add_argument("--stack-block", action="store_true",
                   help="config 4: run each layer as the engine's FFN block (RMSNorm + MoE + residual)")
    p.add_argument("--t1-steps", type=int, default=200)
    p.add_argument("--no-t1", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
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
    return {
        "moe_grouped_gate_up": distinct * gu + T * K * 2 + S * F * 2,
        "moe_grouped_down": distinct * dn + S * F * 2 + S * K * 4,
        "moe_decode_gate_up": distinct * gu + T * K * 4 + S * F * 4,
        # with the certified selection in its prologue: also reads S and B
        "moe_decode_gate_up_sel": distinct * gu + T * K * 4 + S * F * 4 + T * E * (8 + 4),
        "moe_decode_down": distinct * dn + S * F * 4 + T * K * 4,
        "router_logits": W.router_bytes(spec) + T * K * 4 + T * E * 4,
        # certified router: the sums read the router and x, write S, B and the logits;
        # the selection reads S and B
        "router_sums": W.router_bytes(spec) + T * K * 4 + T * E * (8 + 4 + 4),
        "router_select": T * E * (8 + 4),
    }.get(name)


def run_gpu(args, T, steps, warmup, layers, xs, spec, n_used=8):
    """Warmup steps with every kernel timed (per-kernel breakdown, choice of
    the dominant kernel), the timed steps with no per-kernel events, then the
    same steps again with only the dominant kernel bracketed by events.
    Steps are enqueued eagerly: a captured graph of one step's 4-7 kernels
    replays slower than the kernels enqueue (T = 1: 29.4 vs 21.6 us)."""
    from qw3_amd import ds3
    from qw3_amd._native import hip
    E, K = spec.n_expert, spec.n_embd
    out = ds3.Buffer.alloc(T * K * 4)
    idx = ds3.Buffer.alloc(T * n_used * 4)

    def step(i):
        d = layers[i % len(layers)]
        out.zero()
        ds3.moe_ffn_batch(xs[i % len(xs)], d.router, spec.router_type, d.experts, out, T, E, n_used,
                          indices=idx if i == 0 else None)

    step(0)                                   # first touch, routing histogram
    hip().ds3_hip_synchronize()
    counts = np.bincount(idx.read(np.int32, (T, n_used)).reshape(-1), minlength=E)
    hip().ds3_hip_kernel_timing_only(None)
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing(1)
    hip().ds3_hip_begin_batch()
    for i in range(1, warmup + 1):
        step(i)
    hip().ds3_hip_end_batch()
    hip().ds3_hip_kernel_timing(0)
    breakdown = ds3.kernel_stats()
    dominant = max((k for k in breakdown if kernel_bytes(k, spec, T, counts, n_used) is not None),
                   key=lambda k: breakdown[k][1])
    # timed region: synchronise, K steps enqueued back to back, synchronise;
    # no per-kernel events in it (at T = 1 an event pair costs a third of a step)
    hip().ds3_hip_synchronize()
    hip().ds3_hip_begin_batch()
    t0 = time.perf_counter()
    hip().ds3_hip_timer_start()
    for i in range(steps):
        step(i)
    gpu_ms = hip().ds3_hip_timer_stop_ms()
    hip().ds3_hip_end_batch()
    wall_ms = (time.perf_counter() - t0) * 1e3
    # the same K steps again with only the dominant kernel bracketed by
    # events on the library's stream: its average duration for the roofline
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing_only(dominant.encode())
    hip().ds3_hip_kernel_timing(1)
    hip().ds3_hip_begin_batch()
    for i in range(steps):
        step(i)
    hip().ds3_hip_end_batch()
    hip().ds3_hip_kernel_timing(0)
    hip().ds3_hip_kernel_timing_only(None)
    stats = ds3.kernel_stats()
    return wall_ms, gpu_ms, stats, breakdown, counts


def roofline(stats, spec, T, counts, n_used, traffic):
    """traffic: {kernel: HBM bytes per launch} measured at T = 512, and at
    T = 1 under "T1/<kernel>"."""
    name = next(iter(stats))                  # the one kernel timed in the timed region
    n, ms = stats[name]
    avg_s = ms / n / 1e3
    b = kernel_bytes(name, spec, T, counts, n_used)
    achieved = b / avg_s / 1e9
    r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": name,
         "kernel_avg_us": round(avg_s * 1e6, 2), "alg_bytes_per_launch": b}
    key = ("T1/" if T == 1 else "") + name
    if traffic and key in traffic and T in (1, 512):
        r["traffic"] = traffic[key]
    return r


def log_breakdown(brk, stats):
    log("[bench]   warmup, every kernel bracketed by events:")
    for k, (n, ms) in sorted(brk.items(), key=lambda kv: -kv[1][1]):
        log(f"[bench]     {k:24s} {n:5d} launches  avg {ms / n * 1e3:8.2f} us")
    for k, (n, ms) in stats.items():
        log(f"[bench]   timed region, {k} alone: {n} launches avg {ms / n * 1e3:.2f} us")


def cpu_baseline(layer, x, n_used, n_tokens):
    """ds3_ref_moe_ffn (reference build, else the oracle port) per token on
    host threads; ctypes releases the GIL during each call."""
    import concurrent.futures as cf
    import ctypes as C
    sys.path.insert(0, str(ROOT / "tests"))
    import _oracle as O
    spec = layer.spec
    E, K, F = spec.n_expert, spec.n_embd, spec.n_ff
    kind = "reference" if O.ref() is not None else "port"
    deq = O.ref_dequantize if kind == "reference" else O.dequantize
    t0 = time.perf_counter()
    wr = deq(spec.router_type, layer.router, E * K) if spec.router_type != 0 else layer.router.view(np.float32)
    wg = deq(spec.gate_type, layer.gate, E * F * K)
    wu = deq(spec.up_type, layer.up, E * F * K)
    wd = deq(spec.down_type, layer.down, E * K * F)
    log(f"[bench] cpu baseline: dequantised layer in {time.perf_counter() - t0:.1f}s ({kind})")
    fn = O.ref().ds3_ref_moe_ffn if kind == "reference" else O.orc().orc_moe_ffn
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    xt = np.ascontiguousarray(x[:n_tokens])
    out = np.empty_like(xt)

    def work(r):
        lg = np.empty(E, np.float32)
        sc = np.empty(n_used, np.float32)
        ix = np.empty(n_used, np.int32)
        for t in r:
            fn(O.ptr(xt[t]), O.ptr(wr), O.ptr(wg), O.ptr(wu), O.ptr(wd), None, None, None, O.ptr(out[t]),
               O.ptr(lg), O.ptr(sc), O.ptr(ix), K, E, n_used, F, 0, True)

    chunks = [range(i, n_tokens, threads) for i in range(threads)]
    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(threads) as ex:
        list(ex.map(work, chunks))
    dt = time.perf_counter() - t0
    return {"value": round(n_tokens / dt, 2), "unit": "tokens/s", "cores": threads, "kind": kind,
            "sample": f"{n_tokens} tokens of the T={x.shape[0]} batch, one layer, FP32-dequantised weights "
                      f"resident, ds3_ref_moe_ffn per token on {threads} threads ({dt:.1f}s wall)"}


def run_stack(args, n_used=8):
    """Configuration 4: one token per step through a resident stack of
    --stack-layers MoE layers, h <- h + MoE_l(h) in place (the call
    accumulates into its own input), as the engine runs decode.  With
    --stack-block each layer is the engine's whole FFN block instead,
    h <- h + MoE_l(rms_norm(h) * g_l) (ds3_hip_moe_block).  Returns the JSON
    line."""
    from qw3_amd import ds3
    from qw3_amd import workload as W
    from qw3_amd._native import hip
    spec = W.config_spec(4)
    L, K, E = args.stack_layers, spec.n_embd, spec.n_expert
    t0 = time.perf_counter()
    layers = [W.make_layer(spec, seed=1234, layer=l).to_device() for l in range(L)]
    log(f"[bench] config 4: {L} layers generated and resident in {time.perf_counter() - t0:.1f}s "
        f"({L * (W.expert_bytes(spec) * E + W.router_bytes(spec)) / 2**30:.2f} GiB)")
    hs = [ds3.Buffer.from_array(W.make_inputs(4, 1, seed=99, step=s)) for s in range(8)]
    h = ds3.Buffer.alloc(K * 4)
    idx = ds3.Buffer.alloc(n_used * 4)
    gains = [ds3.Buffer.from_array((1.0 + W.fill(W.NORMAL, 700 + l, 1, K, 0.0, 0.02)).astype(np.float32))
             for l in range(L)] if args.stack_block else None

    def token(i, want_idx=False):
        hip().ds3_hip_buffer_copy_f32(hs[i % len(hs)], h, K * 4)     # a fresh hidden state, on the device
        for l, d in enumerate(layers):
            ix = idx if (want_idx and l == 0) else None
            if gains is not None:
                ds3.moe_block(h, gains[l], 1e-6, d.router, spec.router_type, d.experts, 1, E, n_used, indices=ix)
            else:
                ds3.moe_ffn_batch(h, d.router, spec.router_type, d.experts, h, 1, E, n_used, indices=ix)

    token(0, want_idx=True)
    hip().ds3_hip_synchronize()
    counts = np.bincount(idx.read(np.int32, (n_used,)), minlength=E)
    hip().ds3_hip_kernel_timing_only(None)
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing(1)
    hip().ds3_hip_begin_batch()
    for i in range(1, args.warmup + 1):
        token(i)
    hip().ds3_hip_end_batch()
    hip().ds3_hip_kernel_timing(0)
    brk = ds3.kernel_stats()
    dominant = max((k for k in brk if kernel_bytes(k, spec, 1, counts, n_used) is not None),
                   key=lambda k: brk[k][1])
    step = token
    graph = None
    if not args.no_graph:
        # the layers as one HIP graph over h: each token copies its fresh
        # hidden state into h (eagerly), then replays the graph
        graph = ds3.Graph()
        with graph:
            for l, d in enumerate(layers):
                if gains is not None:
                    ds3.moe_block(h, gains[l], 1e-6, d.router, spec.router_type, d.experts, 1, E, n_used)
                else:
                    ds3.moe_ffn_batch(h, d.router, spec.router_type, d.experts, h, 1, E, n_used)

        def step(i):
            hip().ds3_hip_buffer_copy_f32(hs[i % len(hs)], h, K * 4)
            graph.launch()

        hip().ds3_hip_begin_batch()
        for i in range(1, args.warmup + 1):
            step(i)
        hip().ds3_hip_end_batch()
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing_only(dominant.encode())
    # graph replays record no per-kernel events: the dominant kernel is then
    # timed in an eager pass of the same length after the timed region
    hip().ds3_hip_kernel_timing(0 if graph else 1)
    hip().ds3_hip_synchronize()
    hip().ds3_hip_begin_batch()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    hip().ds3_hip_end_batch()
    wall_ms = (time.perf_counter() - t0) * 1e3
    if graph:
        hip().ds3_hip_kernel_timing(1)
        hip().ds3_hip_begin_batch()
        for i in range(args.steps):
            token(i)
        hip().ds3_hip_end_batch()
        graph.close()
    hip().ds3_hip_kernel_timing(0)
    hip().ds3_hip_kernel_timing_only(None)
    stats = ds3.kernel_stats()
    ms = wall_ms / args.steps
    log(f"[bench] config 4: {ms * 1e3:.1f} us/token through {L} layers ({ms * 1e3 / L:.2f} us/layer)"
        + (", layers replayed as one HIP graph" if graph else ""))
    log_breakdown(brk, stats)
    b = L * W.algorithmic_bytes(spec, 1, n_used)
    tpath = Path(args.traffic) if args.traffic else ROOT / "profiles" / "hbm_traffic.json"
    traffic = json.loads(tpath.read_text()) if tpath.exists() else None
    return {
        "metric": f"decode tokens/s through a {L}-layer resident MoE-FFN stack (configs[3]); HBM GB/s vs peak",
        "value": round(1 / (ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded generator; expert weights N(0,0.02) quantised by this project's GGUF quantisers)",
        "config": {"workload": f"configs[3]: decode, one token through {L} resident Qwen3-30B-A3B MoE-FFN layers, "
                               + ("h <- h + MoE_l(rms_norm(h) * g_l) (the engine's FFN block); " if args.stack_block
                                  else "h <- h + MoE_l(h); ")
                               + "Q4_K gate/up + Q6_K down, F32 router"
                               + ("" if args.no_graph else "; layers replayed as one HIP graph"),
                   "tokens": 1, "layers": L, "n_embd": K, "n_ff": spec.n_ff},
        "roofline": roofline(stats, spec, 1, counts, n_used, traffic),
        "alg_bytes_per_step": b,
        "hbm_frac_step": round(b / (ms / 1e3) / (HBM_PEAK_GBS * 1e9), 4),
    }


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
        print(json.dumps(run_stack(args)), flush=True)
        return
    spec = W.config_spec(args.config)
    T, n_used = args.tokens, W.N_USED
    t0 = time.perf_counter()
    hosts, layers = [], []
    for l in range(args.layers):
        h = W.make_layer(spec, seed=1234, layer=l)
        layers.append(h.to_device())
        if l == 0:
            hosts.append(h)
    log(f"[bench] {args.layers} layers generated and resident in {time.perf_counter() - t0:.1f}s")
    xs_host = [W.make_inputs(args.config, T, seed=99, step=s) for s in range(4)]
    xs = [ds3.Buffer.from_array(x) for x in xs_host]

    wall_ms, gpu_ms, stats, brk, counts = run_gpu(args, T, args.steps, args.warmup, layers, xs, spec, n_used)
    ms_step = wall_ms / args.steps
    log(f"[bench] T={T}: {ms_step * 1e3:.1f} us/step wall, {gpu_ms / args.steps * 1e3:.1f} us/step events")
    log_breakdown(brk, stats)
    tpath = Path(args.traffic) if args.traffic else ROOT / "profiles" / "hbm_traffic.json"
    traffic = json.loads(tpath.read_text()) if tpath.exists() else None
    rl = roofline(stats, spec, T, counts, n_used, traffic)
    flops = W.algorithmic_flops(spec, T, n_used)
    line = {
        "metric": "MoE-FFN tokens/s at T=512 (T=1 under t1); HBM GB/s and MFMA util vs peak",
        "value": round(T / (ms_step / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if args.config != 5 else "f16",
        "data": "synthetic (seeded generator; expert weights N(0,0.02) quantised by this project's GGUF quantisers)",
        "config": {"workload": f"configs[{args.config - 1}]: one Qwen3-30B-A3B MoE-FFN layer, T={T} gathered prefill, "
                               f"{W.N_EXPERT} experts top-{n_used}, "
                               f"{ds3.TYPE_NAMES[spec.gate_type]} gate/up + {ds3.TYPE_NAMES[spec.down_type]} down, "
                               f"{ds3.TYPE_NAMES[spec.router_type]} router",
                   "tokens": T, "n_embd": spec.n_embd, "n_ff": spec.n_ff, "layers_cycled": args.layers,
                   "distinct_experts_step0": int((counts > 0).sum())},
        "roofline": rl,
        "mfma_util": round(flops / (ms_step / 1e3) / (FP16_PEAK_TFLOPS * 1e12), 4),
        "alg_bytes_per_step": W.algorithmic_bytes(spec, T, int((counts > 0).sum())),
    }
    line["hbm_frac_step"] = round(line["alg_bytes_per_step"] / (ms_step / 1e3) / (HBM_PEAK_GBS * 1e9), 4)

    if not args.no_t1:
        spec1 = W.config_spec(1)
        layers1 = layers if args.config in (1, 2) else [W.make_layer(spec1, seed=1234, layer=l).to_device()
                                                        for l in range(args.layers)]
        x1 = [ds3.Buffer.from_array(W.make_inputs(1, 1, seed=98, step=s)) for s in range(16)]
        w1, g1, st1, brk1, c1 = run_gpu(args, 1, args.t1_steps, args.warmup, layers1, x1, spec1, n_used)
        ms1 = w1 / args.t1_steps
        log(f"[bench] T=1: {ms1 * 1e3:.1f} us/step wall, {g1 / args.t1_steps * 1e3:.1f} us/step events")
        log_breakdown(brk1, st1)
        b1 = W.algorithmic_bytes(spec1, 1, n_used)
        line["t1"] = {"value": round(1 / (ms1 / 1e3), 1), "unit": "tokens/s", "ms_per_step": round(ms1, 5),
                      "steps": args.t1_steps, "alg_bytes_per_step": b1,
                      "hbm_frac_step": round(b1 / (ms1 / 1e3) / (HBM_PEAK_GBS * 1e9), 4),
                      "roofline": roofline(st1, spec1, 1, c1, n_used, traffic)}

    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(hosts[0], xs_host[0], n_used, min(args.cpu_tokens, T))
        log(f"[bench] cpu baseline {line['cpu_baseline']['value']} tok/s")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
