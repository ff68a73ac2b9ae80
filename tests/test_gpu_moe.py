"""MoE-FFN parity on the GPU, through the C ABI, against the oracle on the
same seeded inputs.

Bars: top-k expert indices identical to the oracle's (its sequential-sum
logits) barring exact ties; combined outputs within max-abs 2e-3 and rel-L2
1e-3 of the FP32 oracle; bucketing identical."""
from contextlib import contextmanager

import numpy as np
import pytest

import _oracle as O
from _cases import Case, assert_close, cert_bound, index_mismatches
from qw3_amd import ds3
from qw3_amd import workload as W
from qw3_amd._native import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def real():
    """Config-1/4 layer: Q4_K gate/up, Q6_K down, FP32 router N(0, 0.02)."""
    print("  building Q4_K/Q6_K layer", flush=True)
    return Case(W.config_spec(1))


@pytest.fixture(scope="module")
def uniform():
    """Config-2 layer: router U(-a, a)."""
    print("  building config-2 layer", flush=True)
    return Case(W.config_spec(2), seed=2024)


@pytest.fixture(scope="module")
def zipf():
    print("  building config-3 layer (Zipf bias)", flush=True)
    return Case(W.config_spec(3), seed=2025)


@pytest.fixture(scope="module")
def q80():
    print("  building config-5 layer (all Q8_0)", flush=True)
    return Case(W.config_spec(5), seed=2026)


def oracle_route(wr: np.ndarray, x: np.ndarray, k: int = W.N_USED, with_logits: bool = False):
    idx = np.empty((x.shape[0], k), np.int32)
    sc = np.empty((x.shape[0], k), np.float32)
    probs = np.empty((x.shape[0], wr.shape[0]), np.float32)
    logits = np.empty((x.shape[0], wr.shape[0]), np.float32)
    for t in range(x.shape[0]):
        logits[t] = O.vec_matmul(x[t], wr)
        idx[t], sc[t], probs[t] = O.route(logits[t], k, with_probs=True)
    return (idx, sc, probs, logits) if with_logits else (idx, sc, probs)


def route_raw(router: ds3.Buffer, rtype: int, x: np.ndarray, E: int, k: int):
    """ds3_hip_moe_route on one router: (indices, scores, logits)."""
    T, K = x.shape
    xb = ds3.Buffer.from_array(x)
    ib, sb, lb = ds3.Buffer.alloc(T * k * 4), ds3.Buffer.alloc(T * k * 4), ds3.Buffer.alloc(T * E * 4)
    ds3.moe_route(xb, router, rtype, T, K, E, k, ib, sb, lb)
    return ib.read(np.int32, (T, k)), sb.read(np.float32, (T, k)), lb.read(np.float32, (T, E))


def gpu_route(case: Case, x: np.ndarray, k: int = W.N_USED):
    return route_raw(case.dev.router, case.spec.router_type, x, case.spec.n_expert, k)


def logit_bits_differ(got: np.ndarray, want: np.ndarray) -> int:
    """Entries whose fp32 bit patterns differ (NaNs compare equal to NaNs)."""
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    return int((~same).sum())


MODES = [ds3.ROUTER_SEQUENTIAL, ds3.ROUTER_CERTIFIED]


@contextmanager
def router_mode(mode: int):
    prev = ds3.set_router_mode(mode)
    try:
        yield
    finally:
        ds3.set_router_mode(prev)


def cert_applies(K: int, E: int) -> bool:
    """Shapes the certified router serves (K a multiple of 256 up to 4096, E <= 256)."""
    return K % 256 == 0 and 256 <= K <= 4096 and E <= 256


def check_logits(gl: np.ndarray, ol: np.ndarray, x: np.ndarray, wr: np.ndarray, mode: int):
    """Sequential router: the reference's logits bit for bit.  Certified
    router: every logit within the proven bound of the reference's (plus its
    own fp32 rounding).  Returns the bound (None for bit-exact)."""
    if mode == ds3.ROUTER_SEQUENTIAL or not cert_applies(x.shape[1], wr.shape[0]):
        assert logit_bits_differ(gl, ol) == 0       # the reference's sequential fp32 sums, bit for bit
        return None
    B = cert_bound(x, wr)
    err = np.abs(gl.astype(np.float64) - ol.astype(np.float64))
    assert (err <= B + np.spacing(np.abs(gl)).astype(np.float64)).all()
    exact = gl.view(np.uint32) == ol.view(np.uint32)
    print(f"    certified logits: max |err|/bound {float(np.max(err / np.maximum(B, 1e-30))):.3f}, "
          f"{exact.mean():.1%} bit-equal", flush=True)
    return B


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("cfg,T", [("real", 64), ("uniform", 512), ("zipf", 2048), ("q80", 256)])
def test_route_indices_bit_exact(hip_ready, request, cfg, T, mode):
    case = request.getfixturevalue(cfg)
    x = W.make_inputs({"real": 1, "uniform": 2, "zipf": 3, "q80": 5}[cfg], T, seed=77)
    print(f"  route {cfg} T={T} mode={mode}", flush=True)
    with router_mode(mode):
        gi, gs, gl = gpu_route(case, x)
    oi, osc, probs, ol = oracle_route(case.wr, x, with_logits=True)
    B = check_logits(gl, ol, x, case.wr, mode)
    assert index_mismatches(gi, oi, probs) == 0
    assert (gi == oi).all()
    rel = np.abs(gs - osc) / np.abs(osc)
    print(f"    weights: max rel diff {rel.max():.2e}", flush=True)
    if B is None:
        # same logits: the weights differ only by the device expf / division roundings
        assert rel.max() < 2e-6
    else:
        # each log-weight moves by at most twice the largest logit bound of its token
        assert (rel <= 2.2 * B.max(axis=1, keepdims=True) + 4e-6).all()


@pytest.mark.parametrize("mode", MODES)
def test_route_near_ties(hip_ready, mode):
    """Router rows 3 and 5 are row 0 shifted by ~1e-8 per element, so their
    logits sit ~5e-7 from row 0's: wider than a probability ulp, inside the
    rounding noise of a reordered fp32 sum.  Only the reference's own
    summation order picks what the reference picks: the certified router
    cannot certify these tokens and must repair them with the exact chains."""
    rng = np.random.default_rng(5)
    wr = (rng.standard_normal((16, 2048)) * 0.02).astype(np.float32)
    x = rng.standard_normal((64, 2048)).astype(np.float32)
    wr[3] = wr[0] + np.float32(1e-8)
    wr[5] = wr[0] - np.float32(1.5e-8)
    with router_mode(mode):
        gi, _, gl = route_raw(ds3.Buffer.from_array(wr), ds3.TYPE_F32, x, 16, 4)
    oi, _, probs, ol = oracle_route(wr, x, 4, with_logits=True)
    check_logits(gl, ol, x, wr, mode)
    assert index_mismatches(gi, oi, probs) == 0
    assert (gi == oi).all()
    if mode == ds3.ROUTER_CERTIFIED:
        # tokens that select expert 0 were repaired: the tied rows carry the exact chains
        sel0 = (oi == 0).any(axis=1)
        assert sel0.sum() > 0
        assert logit_bits_differ(gl[sel0][:, [0, 3, 5]], ol[sel0][:, [0, 3, 5]]) == 0


def _near_tie_router(type_: int, E: int, K: int, rng):
    """Router bytes whose rows 3 and 5 copy row 0 except one weight, moved by
    one code or one fp16 ulp (F32: by 1e-8 per element).  Returns (raw bytes, FP32 rows as the
    oracle dequantises them, index of the changed weight)."""
    if type_ == ds3.TYPE_F32:
        wr = (rng.standard_normal((E, K)) * 0.02).astype(np.float32)
        wr[3] = wr[0] + np.float32(1e-8)
        wr[5] = wr[0] - np.float32(1.5e-8)
        return wr.reshape(-1).view(np.uint8).copy(), wr, None
    if type_ == ds3.TYPE_F16:
        h = (rng.standard_normal((E, K)) * 0.02).astype(np.float16)
        h[3] = h[0]
        h[5] = h[0]
        j = 2048 + 5 if K > 2048 + 5 else 5
        bits = h.view(np.uint16)
        bits[3, j] += 1                       # one fp16 ulp either way
        bits[5, j] -= 1
        return h.reshape(-1).view(np.uint8).copy(), h.astype(np.float32), j
    raw = W.quant_matrix(type_, W.NORMAL, 4321, 7, E, K, 0.0, 0.02).reshape(E, -1).copy()
    raw[3] = raw[0]
    raw[5] = raw[0]
    blk = 1                                   # second block of the row
    if type_ == ds3.TYPE_Q8_0:
        b, j = 34 * blk + 2 + 5, 32 * blk + 5
        for r, dq in ((3, 1), (5, -1)):
            q = int(raw[r, b].astype(np.int8))
            raw[r, b] = np.uint8(np.int8(q + dq if -127 < q + dq < 127 else q - dq))
    elif type_ == ds3.TYPE_Q4_K:
        b, j = 144 * blk + 16 + 32 * 1 + 7, 256 * blk + 64 + 7      # low nibble: weight 64*grp + l
        for r in (3, 5):
            n = int(raw[r, b]) & 15
            raw[r, b] = (int(raw[r, b]) & 0xF0) | (n + 1 if n < 15 else n - 1)
    else:                                     # Q6_K: ql[l] low nibble is weight 128h + l, h = 0
        b, j = 210 * blk + 9, 256 * blk + 9
        for r in (3, 5):
            n = int(raw[r, b]) & 15
            raw[r, b] = (int(raw[r, b]) & 0xF0) | (n + 1 if n < 15 else n - 1)
    raw = raw.reshape(-1)
    wr = O.dequantize(type_, raw, E * K).reshape(E, K)
    return raw, wr, j


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("type_,E", [(ds3.TYPE_F32, 24), (ds3.TYPE_F16, 16), (ds3.TYPE_Q8_0, 16),
                                     (ds3.TYPE_Q8_0, 24), (ds3.TYPE_Q4_K, 16), (ds3.TYPE_Q6_K, 16)])
def test_route_router_types(hip_ready, type_, E, mode):
    """Near ties on every router type, E not a multiple of the 64 experts of
    a wave included: the router rows are expanded to the values of the
    reference's FP32 copy and summed in its order, so logits are bit-exact
    and selection matches the oracle."""
    K, T, k = 2048, 64, 4
    rng = np.random.default_rng(9)
    raw, wr, j = _near_tie_router(type_, E, K, rng)
    x = rng.standard_normal((T, K)).astype(np.float32)
    if j is not None:
        x[:, j] = np.float32(1e-3)            # one code step of that weight moves the logit ~1e-7
    with router_mode(mode):
        gi, _, gl = route_raw(ds3.Buffer.from_array(raw), type_, x, E, k)
    oi, _, probs, ol = oracle_route(wr, x, k, with_logits=True)
    print(f"    {ds3.TYPE_NAMES[type_]} E={E} mode={mode}", flush=True)
    check_logits(gl, ol, x, wr, mode)
    assert index_mismatches(gi, oi, probs) == 0
    assert (gi == oi).all()


@pytest.mark.parametrize("type_", [ds3.TYPE_F32, ds3.TYPE_Q8_0, ds3.TYPE_Q4_K])
def test_moe_ffn_router_logits(hip_ready, type_):
    """ds3_hip_moe_ffn_router (one token): the reference's logits bit for bit."""
    from qw3_amd._native import hip
    K, E = 2048, 128
    rng = np.random.default_rng(21)
    raw, wr, _ = _near_tie_router(type_, E, K, rng)
    x = rng.standard_normal(K).astype(np.float32)
    lb = ds3.Buffer.alloc(E * 4)
    assert hip().ds3_hip_moe_ffn_router(ds3.Buffer.from_array(x), ds3.Buffer.from_array(raw), lb, K, E,
                                        ds3.row_bytes(type_, K), type_) == 0
    assert logit_bits_differ(lb.read(np.float32, (E,)), O.vec_matmul(x, wr)) == 0


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("T,K,E,align", [(1, 2048, 128, 0), (2, 2048, 128, 0), (5, 2048, 128, 0),
                                         (17, 2048, 128, 0), (32, 1000, 72, 0), (37, 1000, 72, 0),
                                         (130, 2048, 128, 4), (1100, 512, 128, 0), (6, 1536, 200, 0),
                                         (3, 4096, 256, 0), (2050, 1024, 136, 0)])
def test_route_logits_shapes(hip_ready, T, K, E, align, mode):
    """Both router kernels (products split off for T <= 32, one lane per
    chain above): ragged T (workgroup tails), K not a multiple of the chunk
    width (scalar tail), E not a multiple of 16, an x row start that is only
    4-byte aligned (4-byte DMAs), and long batches (2-stage ring), also with
    E not a multiple of 16."""
    rng = np.random.default_rng(T + K + E)
    wr = (rng.standard_normal((E, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, K)).astype(np.float32)
    k = 8
    if align:
        # the same rows behind a 4-byte shift: the router reads them through a view
        base = ds3.Buffer.from_array(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)]))
        xb = base.view(align, T * K * 4)
    else:
        xb = ds3.Buffer.from_array(x)
    ib, sb, lb = ds3.Buffer.alloc(T * k * 4), ds3.Buffer.alloc(T * k * 4), ds3.Buffer.alloc(T * E * 4)
    with router_mode(mode):
        ds3.moe_route(xb, ds3.Buffer.from_array(wr), ds3.TYPE_F32, T, K, E, k, ib, sb, lb)
    gl = lb.read(np.float32, (T, E))
    oi, _, probs, ol = oracle_route(wr, x, k, with_logits=True)
    # a 4-byte aligned x row start keeps the sequential router (16-byte loads)
    check_logits(gl, ol, x, wr, ds3.ROUTER_SEQUENTIAL if align else mode)
    assert (ib.read(np.int32, (T, k)) == oi).all()


def test_topk_batch_entry_points(hip_ready):
    rng = np.random.default_rng(11)
    L, T, E, k = 3, 5, 128, 8
    lg = rng.standard_normal((L, T, E)).astype(np.float32)
    lb = ds3.Buffer.from_array(lg)
    ib, sb = ds3.Buffer.alloc(L * T * k * 4), ds3.Buffer.alloc(L * T * k * 4)
    from qw3_amd._native import hip
    assert hip().ds3_hip_moe_router_topk_batch_tokens(lb, ib, sb, L, T, E, k, True) == 0
    gi, gs = ib.read(np.int32, (L, T, k)), sb.read(np.float32, (L, T, k))
    assert hip().ds3_hip_moe_router_topk_batch(lb, ib, sb, L * T, E, k, False) == 0
    gi2, gs2 = ib.read(np.int32, (L * T, k)), sb.read(np.float32, (L * T, k))
    for r in range(L * T):
        oi, osc = O.route(lg.reshape(-1, E)[r], k, norm=True)
        assert np.array_equal(gi.reshape(-1, k)[r], oi)
        assert np.allclose(gs.reshape(-1, k)[r], osc, rtol=2e-6)
        oi2, osc2 = O.route(lg.reshape(-1, E)[r], k, norm=False)
        assert np.array_equal(gi2[r], oi2) and np.allclose(gs2[r], osc2, rtol=2e-6)


# ---------------------------------------------------------------------------
# bucketing
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("T", [1, 37, 512, 2048])
def test_bucket_matches_oracle(hip_ready, T):
    rng = np.random.default_rng(T)
    E, k = 128, 8
    p = rng.random(E) ** 4                      # skewed popularity
    idx = np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)
    sc = rng.random((T, k)).astype(np.float32)
    print(f"  bucket T={T}", flush=True)
    bufs = [ds3.Buffer.alloc(n * 4) for n in (E, E + 1, T * k, T * k, T * k)]
    ds3.moe_bucket(ds3.Buffer.from_array(idx), ds3.Buffer.from_array(sc), T, k, E, *bufs)
    counts, offsets, ids, wts, pos = (b.read(dt, n) for b, dt, n in zip(
        bufs, (np.int32, np.int32, np.int32, np.float32, np.int32), (E, E + 1, T * k, T * k, T * k)))
    oc, oo, oids, owts, opos = O.bucket(idx, sc, E)
    assert np.array_equal(counts, oc) and np.array_equal(offsets[:E], oo) and offsets[E] == T * k
    assert np.array_equal(ids, oids) and np.array_equal(wts, owts) and np.array_equal(pos, opos)


def check_lists(L: dict, idx: np.ndarray, sc: np.ndarray):
    """The grouped path's lists for one chunk (ds3.grouped_lists) against the
    oracle's bucketing of the same routing (reference src/ds3_engine.c:932-955:
    counts, offsets, token ids and weights in token order per expert, the
    position of every slot), bit for bit; then its work items (every expert's
    tiles of tile_m positions in expert order), run lists (every work item
    once per n run, heaviest first: items of 4 m blocks of 16 tokens, then 3,
    2, 1, each class in item order) and the runs' descriptors."""
    E, k, tile_m = L["E"], L["k"], L["tile_m"]
    t0, tc = L["t0"], L["tc"]
    ci, cs = idx[t0:t0 + tc], sc[t0:t0 + tc]
    oc, oo, oids, owts, opos = O.bucket(ci, cs, E)
    assert np.array_equal(L["counts"], oc)
    assert np.array_equal(L["offsets"][:E], oo) and L["offsets"][E] == tc * k
    assert np.array_equal(L["ids"], oids)
    assert np.array_equal(L["wts"].view(np.uint32), owts.view(np.uint32))
    assert np.array_equal(L["slot_pos"], opos)
    want_tiles = [(e << 16) | m for e in range(E) for m in range((int(oc[e]) + tile_m - 1) // tile_m)]
    assert L["tiles"].tolist() == want_tiles
    mb = []                                       # 16-token m blocks of each work item
    for q in want_tiles:
        e, m = q >> 16, q & 0xFFFF
        mb.append((min(tile_m, int(oc[e]) - m * tile_m) + 15) // 16)
    order = [q for c in (4, 3, 2, 1) for q in range(len(want_tiles)) if mb[q] == c]
    for runs, rpi, desc in ((L["runs_gu"], L["rpi_gu"], L["desc_gu"]), (L["runs_dn"], L["rpi_dn"], L["desc_dn"])):
        want_runs = [(q << 12) | j for q in order for j in range(rpi)]
        assert runs.tolist() == want_runs
        # each run's descriptor: its work item's first list position, then
        # expert << 16 | the item's rows << 8 | n run
        want_desc = []
        for q in order:
            e, m = want_tiles[q] >> 16, want_tiles[q] & 0xFFFF
            rows = min(tile_m, int(oc[e]) - m * tile_m)
            want_desc += [[int(oo[e]) + m * tile_m, (e << 16) | (rows << 8) | j] for j in range(rpi)]
        assert desc.tolist() == want_desc


@pytest.mark.parametrize("E,k,T", [(128, 8, 37), (128, 8, 512), (128, 8, 2048), (128, 8, 2050), (48, 8, 300),
                                   (48, 8, 2048), (256, 16, 512), (256, 16, 1000), (64, 6, 101)])
def test_grouped_bucketing_lists(hip_ready, E, k, T):
    """The lists the grouped path builds on the device (the routing's 4-token
    expert bitmaps, then the placement workgroups; past one chunk, chunk by
    chunk) are the oracle's, bit for bit, on the layer's own routing."""
    spec = W.LayerSpec(n_embd=1024, n_ff=256, n_expert=E)
    case = Case(spec, seed=700 + E + k)
    x = W.fill(W.NORMAL, 17, T, T * spec.n_embd, 0.0, 1.0).reshape(T, spec.n_embd)
    print(f"  grouped lists E={E} k={k} T={T}", flush=True)
    got, gi, gs, _ = case.gpu_batch(x, n_used=k, prefill_min=1)
    L = ds3.grouped_lists()
    print(f"    chunk {L['t0']}+{L['tc']}, from bitmaps: {L['marked']}, {len(L['tiles'])} work items", flush=True)
    assert L["marked"]                            # the product path's placement, not the fallback
    assert L["t0"] + L["tc"] == T
    check_lists(L, gi, gs)
    want, oi, osc, probs = case.oracle(x, n_used=k)
    assert index_mismatches(gi, oi, probs) == 0
    assert_close(got, want)


def test_grouped_bucketing_lists_fallback(hip_ready):
    """Router mode 2 routes the grouped path with the certified router, which
    writes no bitmaps: the lists then come from the routed indices (k_bucket),
    and are the same."""
    spec = W.LayerSpec(n_embd=1024, n_ff=256, n_expert=128)
    case = Case(spec, seed=712)
    T = 300
    x = W.fill(W.NORMAL, 18, T, T * spec.n_embd, 0.0, 1.0).reshape(T, spec.n_embd)
    with router_mode(ds3.ROUTER_CERTIFIED):
        _, gi, gs, _ = case.gpu_batch(x, prefill_min=1)
    L = ds3.grouped_lists()
    assert not L["marked"] and L["tc"] == T
    check_lists(L, gi, gs)


@pytest.mark.parametrize("T", [64, 512])
def test_certified_router_grouped_weights(hip_ready, real, T):
    """Router mode 2 on the grouped path: indices the reference's, and the
    routing weights from the exact logits of the selected experts (a launch of
    their sequential chains), so within the device expf / division of the
    oracle's -- not the fp32 rounding of the certified sums."""
    x = W.make_inputs(2, T, seed=117 + T)
    want, oi, osc, probs = real.oracle(x)
    with router_mode(ds3.ROUTER_CERTIFIED):
        got, gi, gs, gl = real.gpu_batch(x, prefill_min=1)
    assert index_mismatches(gi, oi, probs) == 0
    same = (gi == oi).all(axis=1)
    rel = np.abs(gs[same].astype(np.float64) - osc[same]) / osc[same]
    print(f"    weights: max rel err {rel.max():.2e} over {int(same.sum())} rows", flush=True)
    assert rel.max() <= 2e-6
    ol = np.stack([O.vec_matmul(x[t], real.wr) for t in range(T)])
    sel = np.take_along_axis(gl, gi, 1).view(np.uint32)
    assert np.array_equal(sel[same], np.take_along_axis(ol, gi, 1).view(np.uint32)[same])   # exact logits
    assert_close(got, want)


# ---------------------------------------------------------------------------
# full FFN, device-routed
# ---------------------------------------------------------------------------

def test_decode_T1_config1(hip_ready, real):
    """Config 1: single-token decode, 8 independent tokens, one call each."""
    x = W.make_inputs(1, 8, seed=101)
    want, oi, osc, _ = real.oracle(x)
    got = np.empty_like(want)
    for t in range(8):
        print(f"  decode T=1 token {t}", flush=True)
        o, gi, gs, _ = real.gpu_batch(x[t:t + 1])
        assert np.array_equal(gi[0], oi[t])
        got[t] = o[0]
    err, rl = assert_close(got, want)
    assert rl < 5e-5           # the fp32 GEMV path is far inside the bar


def test_prefill_T512_config2(hip_ready, uniform):
    x = W.make_inputs(2, 512, seed=102)
    print("  prefill T=512", flush=True)
    got, gi, gs, _ = uniform.gpu_batch(x)
    want, oi, osc, probs = uniform.oracle(x)
    assert index_mismatches(gi, oi, probs) == 0
    assert_close(got, want)


def test_prefill_T2048_skewed_config3(hip_ready, zipf):
    x = W.make_inputs(3, 2048, seed=103)
    print("  prefill T=2048 skewed", flush=True)
    got, gi, gs, _ = zipf.gpu_batch(x)
    want, oi, osc, probs = zipf.oracle(x)
    assert index_mismatches(gi, oi, probs) == 0
    counts = np.bincount(oi.reshape(-1), minlength=128)
    print(f"    skew: top expert {counts.max()} slots ({counts.max() / oi.size:.1%}), "
          f"{(counts == 0).sum()} experts empty, {((counts >= 1) & (counts <= 2)).sum()} with 1-2", flush=True)
    assert (counts == 0).sum() > 0            # the empty-expert path runs
    assert_close(got, want)


@pytest.mark.parametrize("T", [17, 37, 1000, 2100])
def test_prefill_ragged_and_chunked(hip_ready, uniform, T):
    """Grouped path on token counts that are not multiples of the 16-row MFMA
    blocks or the 64-token tiles, and past one 2048-token bucketing chunk
    (T = 2100: a full chunk, then 52 tokens)."""
    x = W.make_inputs(2, T, seed=110 + T)
    print(f"  prefill ragged T={T}", flush=True)
    got, gi, gs, _ = uniform.gpu_batch(x, prefill_min=1)
    want, oi, osc, probs = uniform.oracle(x)
    assert index_mismatches(gi, oi, probs) == 0
    assert_close(got, want)


def test_prefill_hot_experts(hip_ready):
    """Every token routed to the same 8 experts (router rows of the other
    experts zero, the chosen ones scaled up): 512 tokens give each of them 8
    64-token work items while 120 experts stay empty."""
    hot = np.array([3, 17, 40, 41, 77, 90, 100, 127])
    r = np.zeros((128, 2048), np.float32)
    r[hot] = np.abs(W.fill(W.NORMAL, 77, 5, 8 * 2048, 0.0, 0.02)).reshape(8, 2048)
    x = np.abs(W.make_inputs(2, 512, seed=120)).astype(np.float32)   # hot logits ~ +26, the rest 0
    print("  prefill hot experts T=512", flush=True)
    case = Case(W.LayerSpec(router_dist=W.UNIFORM), seed=77, router=r)
    got, gi, gs, _ = case.gpu_batch(x, prefill_min=1)
    want, oi, osc, probs = case.oracle(x)
    assert set(np.unique(oi).tolist()) == set(hot.tolist())
    assert index_mismatches(gi, oi, probs) == 0
    assert_close(got, want)


@pytest.mark.parametrize("types,offs", [((12, 12, 14), (4, 4, 1)), ((8, 8, 8), (2, 2, 2))])
def test_prefill_unaligned_experts(hip_ready, types, offs):
    """Grouped path on expert tensors whose blocks miss the fast weight loads:
    Q4_K gate and up 4 bytes past a 16-byte boundary (blocks read as dwords
    and realigned), Q6_K down at an odd byte (scales and d in three loads
    instead of two), Q8_0 rows 2 bytes off a dword (every block realigned).
    Same bytes as the oracle's."""
    spec = W.LayerSpec(*types, n_embd=1024, n_ff=256, n_expert=16)
    case = Case(spec, seed=611)
    h = case.host
    keep = []

    def placed(raw, off):
        base = ds3.Buffer.from_array(np.concatenate([np.zeros(off, np.uint8), raw, np.zeros(64, np.uint8)]))
        keep.append(base)
        return base.view(off, raw.nbytes)

    ex = ds3.ExpertTensors(placed(h.gate, offs[0]), placed(h.up, offs[1]), placed(h.down, offs[2]), spec.gate_type,
                           spec.up_type, spec.down_type, spec.n_embd, spec.n_ff)
    T = 96
    x = W.fill(W.NORMAL, 13, T, T * spec.n_embd, 0.0, 1.0).reshape(T, spec.n_embd)
    out = ds3.Buffer.alloc(T * spec.n_embd * 4)
    idx = ds3.Buffer.alloc(T * W.N_USED * 4)
    prev = ds3.set_prefill_min_tokens(1)
    try:
        ds3.moe_ffn_batch(ds3.Buffer.from_array(x), case.dev.router, spec.router_type, ex, out, T, spec.n_expert,
                          W.N_USED, indices=idx)
    finally:
        ds3.set_prefill_min_tokens(prev)
    want, oi, _, probs = case.oracle(x)
    assert index_mismatches(idx.read(np.int32, (T, W.N_USED)), oi, probs) == 0
    assert_close(out.read(np.float32, (T, spec.n_embd)), want)


@pytest.mark.parametrize("E,k,T", [(32, 4, 16), (48, 8, 77), (64, 6, 101), (256, 16, 300)])
def test_prefill_expert_counts(hip_ready, E, k, T):
    """Grouped path (routing with its 4-token expert bitmaps, the parallel
    placement) at other expert counts and top-k widths than Qwen3's: E not
    dividing the placement's 1024 threads (48), up to 256 experts and 16
    slots per token (512 slots per 32-token workgroup), T not a multiple of
    4 or 32."""
    spec = W.LayerSpec(n_embd=1024, n_ff=256, n_expert=E)
    case = Case(spec, seed=600 + E + k)
    x = W.fill(W.NORMAL, 9, T, T * spec.n_embd, 0.0, 1.0).reshape(T, spec.n_embd)
    print(f"  prefill E={E} k={k} T={T}", flush=True)
    got, gi, _, _ = case.gpu_batch(x, n_used=k, prefill_min=1)
    want, oi, _, probs = case.oracle(x, n_used=k)
    assert index_mismatches(gi, oi, probs) == 0
    assert_close(got, want)


@pytest.mark.parametrize("T", [1, 4, 16, 64, 256, 1024])
def test_q8_0_sweep_config5(hip_ready, q80, T):
    x = W.make_inputs(5, T, seed=104 + T)
    print(f"  Q8_0 T={T}", flush=True)
    got, gi, gs, _ = q80.gpu_batch(x)
    want, oi, osc, probs = q80.oracle(x)
    assert index_mismatches(gi, oi, probs) == 0
    assert_close(got, want)


def test_decode_and_prefill_paths_agree(hip_ready, real):
    x = W.make_inputs(2, 64, seed=105)
    want, oi, _, _ = real.oracle(x)
    a, ai, _, _ = real.gpu_batch(x, prefill_min=1 << 30)     # GEMV path
    b, bi, _, _ = real.gpu_batch(x, prefill_min=1)           # grouped MFMA path
    assert np.array_equal(ai, oi) and np.array_equal(bi, oi)
    assert_close(a, want, rel_l2=5e-5)
    assert_close(b, want)


def test_residual_and_accumulate(hip_ready, real):
    """output accumulates into what the caller left there, then + residual
    (reference ds3_metal.h:323 and the engine's residual add, src/ds3_engine.c:1019)."""
    x = W.make_inputs(2, 32, seed=106)
    res = W.fill(W.NORMAL, 3, 99, 32 * 2048, 0.0, 1.0).reshape(32, 2048)
    want, _, _, _ = real.oracle(x)
    for pm in (1, 1 << 30):
        got, _, _, _ = real.gpu_batch(x, residual=res, prefill_min=pm)
        assert_close(got - res, want, max_abs=3e-3, rel_l2=1.2e-3)


@pytest.mark.parametrize("T", [1, 3, 15])
def test_decode_near_ties_fused_select(hip_ready, real, T):
    """Decode with the selection inside the gate/up kernel, on tokens it must
    repair: router rows 3 and 5 are row 0 moved by ~1e-8 per element, and
    every token is pushed towards row 0, so all three sit in its top k
    within the rounding noise of a reordered sum.  Each gate/up workgroup
    re-sums them in the reference's order; the indices, the repaired logits
    and the outputs must match the oracle's."""
    wr = real.wr.copy()
    wr[3] = wr[0] + np.float32(1e-8)
    wr[5] = wr[0] - np.float32(1.5e-8)
    rng = np.random.default_rng(11 + T)
    x = (rng.standard_normal((T, 2048)) + 0.1 * np.sign(wr[0])).astype(np.float32)
    s = real.spec
    want, oi, osc, _ = O.moe_tokens(x, wr, real.wg, real.wu, real.wd, s.n_expert, W.N_USED, s.n_ff, 16, True)
    ol = np.stack([O.vec_matmul(x[t], wr) for t in range(T)])
    assert ((oi == 0).any(axis=1) & (oi == 3).any(axis=1) & (oi == 5).any(axis=1)).all()
    router = ds3.Buffer.from_array(wr)
    xb = ds3.Buffer.from_array(x)
    out, idx = ds3.Buffer.alloc(T * 2048 * 4), ds3.Buffer.alloc(T * W.N_USED * 4)
    sc, lg = ds3.Buffer.alloc(T * W.N_USED * 4), ds3.Buffer.alloc(T * s.n_expert * 4)
    out.zero()
    print(f"  fused-select decode near ties T={T}", flush=True)
    ds3.router_stats(reset=True)
    ds3.moe_ffn_batch(xb, router, ds3.TYPE_F32, real.dev.experts, out, T, s.n_expert, W.N_USED,
                      logits=lg, indices=idx, scores=sc)
    certified, repaired = ds3.router_stats()
    print(f"    router: {certified} certified, {repaired} repaired", flush=True)
    assert repaired == T and certified == 0
    gi, gs, gl = idx.read(np.int32, (T, W.N_USED)), sc.read(np.float32, (T, W.N_USED)), lg.read(np.float32, (T, 128))
    assert np.array_equal(gi, oi)
    assert logit_bits_differ(gl[:, [0, 3, 5]], ol[:, [0, 3, 5]]) == 0
    assert (np.abs(gs - osc) / osc).max() < 1e-5
    assert_close(out.read(np.float32, (T, 2048)), want, rel_l2=5e-5)
    if T == 1:                                       # the single-token entry point takes the same path
        o1, l1 = ds3.Buffer.alloc(2048 * 4), ds3.Buffer.alloc(128 * 4)
        o1.zero()
        ds3.moe_ffn(xb, router, ds3.TYPE_F32, real.dev.experts, o1, l1, s.n_expert, W.N_USED)
        assert logit_bits_differ(l1.read(np.float32, (1, 128))[:, [0, 3, 5]], ol[:, [0, 3, 5]]) == 0
        assert_close(o1.read(np.float32, (1, 2048)), want, rel_l2=5e-5)


@pytest.fixture(scope="module")
def wide_router():
    """Q4_K/Q6_K layer (n_ff 256) whose F32 router rows and inputs are
    U(-0.5, 0.5), as in the reference's tests/test_moe_metal.c:148-156:
    logits ~ N(0, 3.8), so the reference's chain lands ~1e-5 from the exact
    sum and weights from fl32(S) would be ~1e-5 off."""
    spec = W.LayerSpec(n_ff=256)
    router = W.fill(W.UNIFORM, 31, 1, spec.n_expert * spec.n_embd, -0.5, 0.5).reshape(spec.n_expert, spec.n_embd)
    print("  building wide-router layer", flush=True)
    return Case(spec, seed=3131, router=router)


@pytest.mark.parametrize("T", [1, 2, 12])
def test_certified_weights_from_exact_logits(hip_ready, wide_router, T):
    """Certified decode routing (T = 1 fused selection, T = 2 .. 12 the
    selection launch): indices the reference's, the selected experts' logits
    bit for bit the reference's sequential chains, and the weights those
    logits give (within the device expf / division roundings)."""
    case, s = wide_router, wide_router.spec
    x = W.fill(W.UNIFORM, 40 + T, 2, T * s.n_embd, -0.5, 0.5).reshape(T, s.n_embd)
    oi, osc, _, ol = oracle_route(case.wr, x, with_logits=True)
    ds3.router_stats(reset=True)
    print(f"  certified weights T={T}", flush=True)
    got, gi, gs, gl = case.gpu_batch(x)
    certified, repaired = ds3.router_stats()
    print(f"    router: {certified} certified, {repaired} repaired", flush=True)
    assert certified + repaired == T and certified >= T - 2      # a close pair may still send a token to repair
    assert np.array_equal(gi, oi)
    sel = np.take_along_axis(gl, gi, axis=1)
    assert logit_bits_differ(sel, np.take_along_axis(ol, oi, axis=1)) == 0
    rel = np.abs(gs - osc) / osc
    print(f"    weights: max rel diff {rel.max():.2e}", flush=True)
    assert rel.max() < 2e-6
    want, _, _, _ = case.oracle(x)
    assert_close(got, want, rel_l2=5e-5)
    if T == 1:                                       # the single-token entry point
        o1, l1 = ds3.Buffer.alloc(s.n_embd * 4), ds3.Buffer.alloc(s.n_expert * 4)
        o1.zero()
        ds3.moe_ffn(ds3.Buffer.from_array(x), case.dev.router, ds3.TYPE_F32, case.dev.experts, o1, l1, s.n_expert,
                    W.N_USED)
        l1h = l1.read(np.float32, (1, s.n_expert))
        assert logit_bits_differ(np.take_along_axis(l1h, oi, axis=1), np.take_along_axis(ol, oi, axis=1)) == 0
        assert_close(o1.read(np.float32, (1, s.n_embd)), want, rel_l2=5e-5)


@pytest.mark.parametrize("n_embd,n_ff,n_expert,n_used", [
    (1024, 256, 32, 4),       # one Q6_K superblock per down row
    (1024, 512, 32, 8),
    (2048, 1024, 32, 8),      # four superblocks per down row, 87 KiB of staged rows per workgroup
    (1024, 1024, 32, 16),     # 16 slots would need 173 KiB of LDS: the unstaged down kernel
])
def test_decode_down_shapes(hip_ready, n_embd, n_ff, n_expert, n_used):
    """Decode (T = 1 fused selection + L2 warm-up, T = 3 separate selection)
    on Q4_K gate/up and Q6_K down of other widths and slot counts than
    Qwen3's, through the staged and unstaged down kernels."""
    spec = W.LayerSpec(n_embd=n_embd, n_ff=n_ff, n_expert=n_expert)
    case = Case(spec, seed=500 + n_ff + n_used)
    for T in (1, 3):
        x = W.fill(W.NORMAL, 7, T, T * n_embd, 0.0, 1.0).reshape(T, n_embd)
        want, oi, _, probs = case.oracle(x, n_used=n_used)
        print(f"  decode {n_embd}x{n_ff} E={n_expert} k={n_used} T={T}", flush=True)
        got, gi, _, _ = case.gpu_batch(x, n_used=n_used)
        assert index_mismatches(gi, oi, probs) == 0
        assert_close(got, want, rel_l2=5e-5)


def test_decode_stack_teacher_forced_config4(hip_ready):
    """Configuration 4 in small: h <- h + MoE_l(h) through distinct layers at
    T = 1 (decode path, residual fused), each layer checked against the
    oracle on the oracle's own input (teacher forcing), for a few steps of
    fresh tokens."""
    spec = W.config_spec(4)
    cases = [Case(spec, seed=1234, layer=l) for l in range(3)]
    for step in range(2):
        h = W.make_inputs(4, 1, seed=99, step=step)
        for l, case in enumerate(cases):
            want, oi, _, probs = case.oracle(h)
            want = want + h                                 # residual (reference src/ds3_reference.c:455-460)
            print(f"  stack step {step} layer {l}", flush=True)
            got, gi, _, _ = case.gpu_batch(h, residual=h)
            assert index_mismatches(gi, oi, probs) == 0
            assert_close(got, want, max_abs=3e-3, rel_l2=1.2e-3)
            h = want                                        # teacher forcing


# ---------------------------------------------------------------------------
# ds3_metal.h entry points (reference tests/test_moe_metal.c cases)
# ---------------------------------------------------------------------------

def _metal_case(name, n_embd, n_expert, n_used, n_ff, gt, ut, dt, tol, seed):
    spec = W.LayerSpec(gt, ut, dt, ds3.TYPE_F32, W.UNIFORM, 0.5 / np.sqrt(3), n_embd, n_ff, n_expert)
    case = Case(spec, seed=seed)
    x = W.fill(W.UNIFORM, seed, 1, n_embd, -0.5, 0.5).reshape(1, n_embd)
    want, oi, _, _ = case.oracle(x, n_used=n_used)
    out = ds3.Buffer.alloc(n_embd * 4)
    out.zero()
    logits = ds3.Buffer.alloc(n_expert * 4)
    print(f"  moe_ffn {name}", flush=True)
    ds3.moe_ffn(ds3.Buffer.from_array(x), case.dev.router, ds3.TYPE_F32, case.dev.experts, out, logits,
                n_expert, n_used)
    got = out.read(np.float32, (1, n_embd))
    assert float(np.abs(got - want).max()) < tol
    return case, x, want


@pytest.mark.parametrize("name,shape,types,tol", [
    ("small_f32", (256, 16, 4, 128), (0, 0, 0), 1e-3),            # test_moe_metal.c:26-118
    ("qwen3_dims_f32", (2048, 128, 8, 768), (0, 0, 0), 1e-3),    # :120-212
    ("qwen3_dims_q4k", (2048, 128, 8, 768), (12, 12, 12), 2e-3),  # :214-365
    ("qwen3_dims_mixed", (2048, 128, 8, 768), (12, 12, 0), 2e-3),  # :369-505
    ("qwen3_dims_q4k_q6k", (2048, 128, 8, 768), (12, 12, 14), 2e-3),  # :509-659
    ("q4k_gate_q8_up", (2048, 32, 4, 768), (12, 8, 14), 2e-3),    # mixed gate/up types: unfused fallback
])
def test_moe_ffn_entry_point(hip_ready, name, shape, types, tol):
    _metal_case(name, *shape, *types, tol, seed=70 + len(name))


def test_moe_ffn_experts_host_indices(hip_ready, real):
    x = W.make_inputs(1, 1, seed=107)
    want, oi, osc, _ = real.oracle(x)
    out = ds3.Buffer.alloc(2048 * 4)
    out.zero()
    scratch = ds3.Buffer.alloc(768 * 4)
    gs, us, dsd = real.dev.experts.strides
    from qw3_amd._native import hip
    import ctypes as C
    ii = np.ascontiguousarray(oi[0], np.int32)
    ss = np.ascontiguousarray(osc[0], np.float32)
    rc = hip().ds3_hip_moe_ffn_experts(
        ds3.Buffer.from_array(x), real.dev.experts.gate, real.dev.experts.up,
        real.dev.experts.down, 12, 12, 14, gs, us, dsd, None, None, None, 0, 0, 0, 0, 0, 0,
        out, scratch, scratch, scratch, 2048, 8, 768, 0,
        ii.ctypes.data_as(C.POINTER(C.c_int32)), ss.ctypes.data_as(C.POINTER(C.c_float)))
    assert rc == 0
    assert_close(out.read(np.float32, (1, 2048)), want, rel_l2=1e-5)


def test_expert_offset_table(hip_ready, real):
    """expert_offsets [E][3] (reference ds3_metal.h:325-329) addresses the same bytes."""
    gs, us, dsd = real.dev.experts.strides
    tbl = np.array([[e * 768 * gs, e * 768 * us, e * 2048 * dsd] for e in range(128)], np.uint64)
    x = W.make_inputs(2, 48, seed=108)
    want, _, _, _ = real.oracle(x)
    for pm in (1, 1 << 30):                     # grouped MFMA path, then the GEMV path
        T = 48
        out = ds3.Buffer.alloc(T * 2048 * 4)
        prev = ds3.set_prefill_min_tokens(pm)
        try:
            ds3.moe_ffn_batch(ds3.Buffer.from_array(x), real.dev.router, 0, real.dev.experts, out, T, 128, 8,
                              expert_offsets=ds3.Buffer.from_array(tbl))
        finally:
            ds3.set_prefill_min_tokens(prev)
        assert_close(out.read(np.float32, (T, 2048)), want, rel_l2=1e-3 if pm == 1 else 5e-5)


def test_shared_expert(hip_ready):
    K, E, k, Fd, Fs = 512, 16, 4, 256, 768
    spec = W.LayerSpec(12, 12, 14, 0, W.NORMAL, 0.05, K, Fd, E)
    case = Case(spec, seed=9)
    sh = Case(W.LayerSpec(12, 12, 14, 0, W.NORMAL, 0.05, K, Fs, 1), seed=10)
    x = W.fill(W.NORMAL, 1, 1, K, 0.0, 1.0).reshape(1, K)
    out_ref = np.empty(K, np.float32)
    lg, sc, idx = np.empty(E, np.float32), np.empty(k, np.float32), np.empty(k, np.int32)
    O.orc().orc_moe_ffn(O.ptr(x), O.ptr(case.wr), O.ptr(case.wg), O.ptr(case.wu), O.ptr(case.wd),
                        O.ptr(sh.wg), O.ptr(sh.wu), O.ptr(sh.wd), O.ptr(out_ref), O.ptr(lg), O.ptr(sc), O.ptr(idx),
                        K, E, k, Fd, Fs, True)
    out = ds3.Buffer.alloc(K * 4)
    out.zero()
    ds3.moe_ffn(ds3.Buffer.from_array(x), case.dev.router, 0, case.dev.experts, out, ds3.Buffer.alloc(E * 4), E, k,
                shared=sh.dev.experts, n_ff_shared=Fs)
    assert_close(out.read(np.float32, (1, K)), out_ref.reshape(1, K), rel_l2=1e-5)


# ---------------------------------------------------------------------------
# products and elementwise entry points
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("t,M,N,K,tol", [(8, 32, 128, 256, 2e-4), (12, 16, 64, 256, 2e-4), (14, 16, 64, 256, 3e-4),
                                         (12, 1, 4096, 2048, 2e-4), (14, 33, 2048, 768, 3e-4)])
def test_matmul_quantized_batch(hip_ready, t, M, N, K, tol):
    """Reference tests/test_matmul_quant_metal.c:633-907 tolerances."""
    rng = np.random.default_rng(M * N + K)
    A = (rng.random((M, K)) - 0.5).astype(np.float32)
    raw = W.quant_matrix(t, W.UNIFORM, 3, t, N, K, -0.5, 0.5)
    Wf = O.dequantize(t, raw, N * K).reshape(N, K)
    want = np.stack([O.vec_matmul(A[m], Wf) for m in range(M)])
    wb = ds3.Buffer.alloc(raw.nbytes + 512)
    wb.write(raw, offset=512)
    cb = ds3.Buffer.alloc(M * N * 4)
    from qw3_amd._native import hip
    assert hip().ds3_hip_matmul_quantized_batch(ds3.Buffer.from_array(A), wb, cb, M, N, K,
                                                ds3.row_bytes(t, K), 512, t) == 0
    assert float(np.abs(cb.read(np.float32, (M, N)) - want).max()) < tol


@pytest.mark.parametrize("t", [8, 12, 14])
def test_vec_matmul_quantized(hip_ready, t):
    rng = np.random.default_rng(t)
    x = (rng.random(2048) - 0.5).astype(np.float32)
    raw = W.quant_matrix(t, W.UNIFORM, 4, t, 1024, 2048, -0.5, 0.5)
    want = O.vec_matmul(x, O.dequantize(t, raw, 1024 * 2048).reshape(1024, 2048))
    yb = ds3.Buffer.alloc(1024 * 4)
    from qw3_amd._native import hip
    fn = {8: "q8_0", 12: "q4k", 14: "q6k"}[t]
    assert hip().ds3_hip_vec_matmul_quantized(ds3.Buffer.from_array(x), ds3.Buffer.from_array(raw),
                                              yb, 2048, 1024, ds3.row_bytes(t, 2048), t) == 0
    assert float(np.abs(yb.read(np.float32, 1024) - want).max()) < 1e-4
    assert getattr(hip(), f"ds3_hip_vec_matmul_{fn}_simd")(ds3.Buffer.from_array(x),
                                                           ds3.Buffer.from_array(raw), yb, 2048, 1024,
                                                           ds3.row_bytes(t, 2048)) == 0
    assert float(np.abs(yb.read(np.float32, 1024) - want).max()) < 1e-4


def test_elementwise_entry_points(hip_ready):
    from qw3_amd._native import hip
    rng = np.random.default_rng(2)
    n, cols, count = 4096, 64, 20
    a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    ab, bb, cb = ds3.Buffer.from_array(a), ds3.Buffer.from_array(b), ds3.Buffer.alloc(n * 4)
    assert hip().ds3_hip_vec_add(ab, bb, cb, n) == 0
    assert np.array_equal(cb.read(np.float32, n), a + b)
    assert hip().ds3_hip_vec_add_inplace(ab, bb, n) == 0
    assert np.array_equal(ab.read(np.float32, n), a + b)
    assert hip().ds3_hip_buffer_copy_f32(bb, cb, n * 4) == 0
    assert np.array_equal(cb.read(np.float32, n), b)
    assert hip().ds3_hip_buffer_zero_f32(cb, n * 4) == 0
    assert not cb.read(np.float32, n).any()
    assert hip().ds3_hip_silu_mul_f32(bb, ds3.Buffer.from_array(a), cb, n) == 0
    want = np.empty(n, np.float32)
    O.orc().orc_silu(O.ptr(b), O.ptr(want), n)
    assert np.allclose(cb.read(np.float32, n), want * a, rtol=2e-6, atol=1e-7)
    src = rng.standard_normal((50, cols)).astype(np.float32)
    ids = np.array([7] + list(rng.choice(50, count, replace=False)), np.int32)
    sc = np.concatenate([[9.0], rng.random(count)]).astype(np.float32)
    dst = ds3.Buffer.alloc(count * cols * 4)
    assert hip().ds3_hip_gather_rows_f32(ds3.Buffer.from_array(src), ds3.Buffer.from_array(ids),
                                         dst, cols, count, 1) == 0
    g = dst.read(np.float32, (count, cols))
    assert np.array_equal(g, src[ids[1:]])
    base = rng.standard_normal((50, cols)).astype(np.float32)
    db = ds3.Buffer.from_array(base)
    assert hip().ds3_hip_scatter_add_weighted_f32(dst, ds3.Buffer.from_array(sc),
                                                  ds3.Buffer.from_array(ids), db, cols, count, 1) == 0
    want = base.copy()
    want[ids[1:]] += sc[1:, None] * g
    assert np.allclose(db.read(np.float32, (50, cols)), want, rtol=1e-6, atol=1e-6)


def test_invalid_arguments_return_error(hip_ready, real):
    """Argument rules of reference src/ds3_metal.m:1841-1862, 2453-2485:
    -1 and output untouched."""
    from qw3_amd._native import hip
    x = ds3.Buffer.from_array(np.ones(2048, np.float32))
    out = ds3.Buffer.from_array(np.full(2048, 7.0, np.float32))
    lg = ds3.Buffer.alloc(128 * 4)
    s = ds3.Buffer.alloc(4096)
    e = real.dev.experts
    gs, us, dsd = e.strides

    def call(gt=12, ut=12, dt=14, n_embd=2048, n_used=8, n_expert=128, n_ff=768, eu=s, ed=s, rt=0):
        return hip().ds3_hip_moe_ffn(x, real.dev.router, e.gate, e.up, e.down,
                                     gt, ut, dt, gs, us, dsd, None, None, None, 0, 0, 0, 0, 0, 0,
                                     out, lg, None, s, eu and eu, ed and ed,
                                     n_embd, n_expert, n_used, n_ff, 0, 2048 * 4, rt, True)
    assert call(gt=99) == -1                    # unsupported type
    assert call(dt=14, n_ff=700) == -1           # K-quant in_dim % 256
    assert call(n_used=129) == -1               # n_used > n_expert
    assert call(n_used=0) == -1
    assert call(eu=None) == -1                  # quantised path needs expert_up/expert_down
    assert np.all(out.read(np.float32, 2048) == 7.0)
    assert hip().ds3_hip_matmul_quantized_batch(x, e.gate, out, 1, 4, 100, 144, 0, 12) == -1
    assert hip().ds3_hip_buffer_zero_f32(out, 6) == -1
    assert hip().ds3_hip_dequantize(x, 0, 12, 100, out) == -1


def test_short_weight_buffers_return_error(hip_ready, real):
    """Every MoE entry point refuses weights that do not hold what the call
    would read on the device -- a router of fewer than n_expert rows, expert
    tensors of fewer than n_expert experts, row strides shorter than a row, an
    offset table of fewer than n_expert x 3 entries -- with -1 and the output
    untouched, rather than reading past the buffer."""
    d, e = real.dev, real.dev.experts
    gs, us, dsd = e.strides
    E, K, F = 128, 2048, 768
    router = d.router
    short_router = router.view(0, (E - 1) * K * 4)
    short_gate = e.gate.view(0, (E - 1) * F * gs)
    short_down = e.down.view(0, E * K * dsd - 1)
    short_table = ds3.Buffer.alloc(E * 3 * 8 - 8)
    full_table = ds3.Buffer.from_array(
        np.array([[i * F * gs, i * F * us, i * K * dsd] for i in range(E)], np.uint64))
    for T in (1, 64):
        x = ds3.Buffer.from_array(W.make_inputs(2, T, seed=115))
        out = ds3.Buffer.from_array(np.full(T * K, 7.0, np.float32))

        def batch(fn, rt=router, g=e.gate, dn=e.down, gst=gs, table=None, rstride=K * 4):
            return fn(x, rt, g, e.up, dn, 12, 12, 14, gst, us, dsd, table, out, None, None, None, None,
                      T, K, E, 8, F, rstride, 0, True)

        def block(rt=router, g=e.gate, dn=e.down, gst=gs, table=None, rstride=K * 4):
            gain = ds3.Buffer.from_array(np.ones(K, np.float32))
            return hip_fn("ds3_hip_moe_block")(out, gain, 1e-6, rt, g, e.up, dn, 12, 12, 14, gst, us, dsd, table,
                                               None, None, None, None, T, K, E, 8, F, rstride, 0, True)

        for fn in (hip_fn("ds3_hip_moe_ffn_batch"), hip_fn("ds3_hip_moe_ffn_batch_noalloc")):
            print(f"  T={T} {fn.__name__}", flush=True)
            assert batch(fn, rt=short_router) == -1
            assert batch(fn, g=short_gate) == -1
            assert batch(fn, dn=short_down) == -1
            assert batch(fn, gst=gs - 1) == -1
            assert batch(fn, rstride=K * 4 - 4) == -1
            assert batch(fn, table=short_table) == -1
        assert block(rt=short_router) == -1
        assert block(g=short_gate) == -1
        assert block(table=short_table) == -1
        assert np.all(out.read(np.float32, T * K) == 7.0)
        # a full table and full-size weights go through
        assert batch(hip_fn("ds3_hip_moe_ffn_batch"), table=full_table) == 0
    x1 = ds3.Buffer.from_array(W.make_inputs(1, 1, seed=116))
    out1 = ds3.Buffer.from_array(np.full(K, 7.0, np.float32))
    lg = ds3.Buffer.alloc(E * 4)
    scr = ds3.Buffer.alloc(4096)

    def moe_ffn(rt=router, g=e.gate, dn=e.down, table=None):
        return hip_fn("ds3_hip_moe_ffn")(x1, rt, g, e.up, dn, 12, 12, 14, gs, us, dsd, None, None, None, 0, 0, 0,
                                         0, 0, 0, out1, lg, table, scr, scr, scr, K, E, 8, F, 0, K * 4, 0, True)
    assert moe_ffn(rt=short_router) == -1
    assert moe_ffn(g=short_gate) == -1
    assert moe_ffn(dn=short_down) == -1
    assert moe_ffn(table=short_table) == -1
    assert np.all(out1.read(np.float32, K) == 7.0)
    assert moe_ffn() == 0


def hip_fn(name):
    from qw3_amd._native import hip
    return getattr(hip(), name)


# ---------------------------------------------------------------------------
# FFN block: RMSNorm prologue + MoE + residual in one call
# ---------------------------------------------------------------------------

def test_rms_norm_entry_point(hip_ready):
    """reference tests/test_metal.c:32-80: 4 rows of 2048 from C rand() with
    srand(42), weight 1 + (rand() % 100) / 1000, eps 1e-6; the reference's
    bar is max |diff| < 1e-4 against ds3_ref_rms_norm; also the ulp bounds
    of check_norm_ulps (only the order of the sum of squares differs)."""
    import ctypes
    libc = ctypes.CDLL("libc.so.6")
    libc.srand(42)
    n, rows, eps = 2048, 4, 1e-6
    x = np.array([(libc.rand() % 1000) / 1000.0 - 0.5 for _ in range(rows * n)], np.float32).reshape(rows, n)
    w = np.array([1.0 + (libc.rand() % 100) / 1000.0 for _ in range(n)], np.float32)
    want = O.rms_norm(x, w, eps)
    out = ds3.Buffer.alloc(rows * n * 4)
    ds3.rms_norm(ds3.Buffer.from_array(x), ds3.Buffer.from_array(w), out, n, rows, eps)
    got = out.read(np.float32, (rows, n))
    assert float(np.abs(got - want).max()) < 1e-4
    check_norm_ulps(got, x, w, eps, want)


@pytest.mark.parametrize("n,rows", [(64, 3), (300, 2), (2048, 5), (4000, 2)])
def test_rms_norm_shapes(hip_ready, n, rows):
    """Row lengths that are not a multiple of the 256-thread workgroup (runs of
    ceil(n / 256) elements per thread, the last threads idle), each row in a
    workgroup of its own; same bounds as above."""
    x = W.fill(W.NORMAL, 40 + n, rows, rows * n, 0.0, 1.0).reshape(rows, n)
    w = (1.0 + W.fill(W.NORMAL, 41 + n, 1, n, 0.0, 0.02)).astype(np.float32)
    out = ds3.Buffer.alloc(rows * n * 4)
    print(f"  rms_norm n={n} rows={rows}", flush=True)
    ds3.rms_norm(ds3.Buffer.from_array(x), ds3.Buffer.from_array(w), out, n, rows, 1e-6)
    check_norm_ulps(out.read(np.float32, (rows, n)), x, w, 1e-6, O.rms_norm(x, w, 1e-6))


def check_norm_ulps(got: np.ndarray, x: np.ndarray, w: np.ndarray, eps: float, want: np.ndarray):
    """got within 8 ulp of the formula in float64 (the tree sum of squares
    rounds about log2(n) times) and within 64 ulp of the reference's result,
    whose 2048-term left-to-right sum carries ~sqrt(n) ulp of rounding noise."""
    xd = x.astype(np.float64)
    exact = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)
    sp = np.spacing(np.abs(got)).astype(np.float64)
    u_exact = np.abs(got - exact) / sp
    u_ref = np.abs(got.astype(np.float64) - want) / sp
    print(f"    rms_norm: {u_exact.max():.1f} ulp from float64, {u_ref.max():.1f} ulp from the reference", flush=True)
    assert u_exact.max() <= 8
    assert u_ref.max() <= 64


@pytest.mark.parametrize("T", [1, 2, 3, 16, 64])
def test_moe_block(hip_ready, real, T):
    """hidden += MoE(rms_norm(hidden) * g) in place (reference engine
    src/ds3_engine.c:519-527, 675-720), on the decode (T = 1 fused selection,
    T = 2, 3, 16) and grouped (T = 64) paths.  Up to 16 tokens the certified
    router's sums kernel normalises the rows itself; its x_norm must equal
    the rms_norm entry point's bit for bit, and is checked as rms_norm's is.
    The MoE is checked against the oracle run on those rows (indices exact,
    outputs to the decode or grouped bar), and a second call without x_norm
    gives the same hidden."""
    s = real.spec
    hid = W.fill(W.NORMAL, 31, T, T * s.n_embd, 0.0, 1.0).reshape(T, s.n_embd)
    g = (1.0 + W.fill(W.NORMAL, 32, 1, s.n_embd, 0.0, 0.02)).astype(np.float32)
    eps = 1e-6
    hb, gb = ds3.Buffer.from_array(hid), ds3.Buffer.from_array(g)
    xn = ds3.Buffer.alloc(T * s.n_embd * 4)
    idx = ds3.Buffer.alloc(T * W.N_USED * 4)
    print(f"  moe_block T={T}", flush=True)
    ds3.moe_block(hb, gb, eps, real.dev.router, s.router_type, real.dev.experts, T, s.n_expert, W.N_USED,
                  x_norm=xn, indices=idx)
    got_xn = xn.read(np.float32, (T, s.n_embd))
    sep = ds3.Buffer.alloc(T * s.n_embd * 4)
    ds3.rms_norm(ds3.Buffer.from_array(hid), gb, sep, s.n_embd, T, eps)
    assert np.array_equal(got_xn.view(np.uint32), sep.read(np.float32, (T, s.n_embd)).view(np.uint32))
    check_norm_ulps(got_xn, hid, g, eps, O.rms_norm(hid, g, eps))
    want, oi, _, probs = real.oracle(got_xn)
    assert index_mismatches(idx.read(np.int32, (T, W.N_USED)), oi, probs) == 0
    after = hb.read(np.float32, (T, s.n_embd))
    assert_close(after - hid, want, rel_l2=5e-5 if T < 16 else 1e-3)
    hb2 = ds3.Buffer.from_array(hid)
    ds3.moe_block(hb2, gb, eps, real.dev.router, s.router_type, real.dev.experts, T, s.n_expert, W.N_USED)
    assert np.array_equal(hb2.read(np.float32, (T, s.n_embd)), after)


@pytest.mark.parametrize("T", [1, 5, 64])
def test_moe_ffn_batch_in_place(hip_ready, real, T):
    """output may be the input itself: h += MoE(h) with no zeroed output and
    no residual gives what output = 0, residual = h gives (the same sums,
    added to h in another order: within a few fp32 roundings)."""
    s = real.spec
    hid = W.fill(W.NORMAL, 51, T, T * s.n_embd, 0.0, 1.0).reshape(T, s.n_embd)
    print(f"  moe_ffn_batch in place T={T}", flush=True)
    xb, out = ds3.Buffer.from_array(hid), ds3.Buffer.alloc(T * s.n_embd * 4)
    out.zero()
    ds3.moe_ffn_batch(xb, real.dev.router, s.router_type, real.dev.experts, out, T, s.n_expert, W.N_USED,
                      residual=xb)
    want = out.read(np.float32, (T, s.n_embd))
    hb = ds3.Buffer.from_array(hid)
    ds3.moe_ffn_batch(hb, real.dev.router, s.router_type, real.dev.experts, hb, T, s.n_expert, W.N_USED)
    got = hb.read(np.float32, (T, s.n_embd))
    # h + (w_1 y_1 + ...) rounds after each of the 8 adds at |h|'s scale instead of once
    np.testing.assert_allclose(got, want, rtol=0, atol=8 * float(np.spacing(np.abs(want).max())))


@pytest.mark.parametrize("T", [1, 64])
def test_graph_replay(hip_ready, real, T):
    """A captured zero + moe_ffn_batch (decode path with the fused selection at
    T = 1, grouped path at T = 64) replayed three times, with eager calls on
    other buffers and synchronisations between the replays: every replay
    rewrites the poisoned output with exactly the eager result."""
    from qw3_amd._native import hip
    s = real.spec
    xb = ds3.Buffer.from_array(W.make_inputs(2, T, seed=130))
    out, idx = ds3.Buffer.alloc(T * s.n_embd * 4), ds3.Buffer.alloc(T * W.N_USED * 4)
    xo, oo = ds3.Buffer.from_array(W.make_inputs(2, T, seed=131)), ds3.Buffer.alloc(T * s.n_embd * 4)

    def call(x, o, ix=None):
        o.zero()                                   # a fill kernel, not a memset node
        ds3.moe_ffn_batch(x, real.dev.router, s.router_type, real.dev.experts, o, T, s.n_expert, W.N_USED,
                          indices=ix)

    print(f"  graph replay T={T}", flush=True)
    call(xb, out, idx)
    want, want_i = out.read(np.float32, (T, s.n_embd)), idx.read(np.int32, (T, W.N_USED))
    call(xo, oo)
    want_o = oo.read(np.float32, (T, s.n_embd))
    with ds3.Graph() as gr:
        call(xb, out, idx)
    try:
        for rep in range(3):
            out.write(np.full((T, s.n_embd), 7.0, np.float32))
            idx.write(np.full((T, W.N_USED), -1, np.int32))
            gr.launch()
            assert np.array_equal(out.read(np.float32, (T, s.n_embd)), want), f"replay {rep}"
            assert np.array_equal(idx.read(np.int32, (T, W.N_USED)), want_i), f"replay {rep}"
            call(xo, oo)                           # eager work between the replays
            hip().ds3_hip_synchronize()
            assert np.array_equal(oo.read(np.float32, (T, s.n_embd)), want_o)
    finally:
        gr.close()


# ---------------------------------------------------------------------------
# read-only routers: the FP32 copy made once
# ---------------------------------------------------------------------------

def _batch_run(dev, spec, x, n_used=8):
    T = x.shape[0]
    out = ds3.Buffer.alloc(T * spec.n_embd * 4)
    idx = ds3.Buffer.alloc(T * n_used * 4)
    sc = ds3.Buffer.alloc(T * n_used * 4)
    lg = ds3.Buffer.alloc(T * spec.n_expert * 4)
    hip().ds3_hip_kernel_timing_reset()
    hip().ds3_hip_kernel_timing(1)
    ds3.moe_ffn_batch(ds3.Buffer.from_array(x), dev.router, spec.router_type, dev.experts, out, T, spec.n_expert,
                      n_used, logits=lg, indices=idx, scores=sc)
    hip().ds3_hip_kernel_timing(0)
    ran = set(ds3.kernel_stats())
    return (out.read(np.float32, (T, spec.n_embd)), idx.read(np.int32, (T, n_used)), sc.read(np.float32, (T, n_used)),
            lg.read(np.float32, (T, spec.n_expert))), ran


def test_readonly_router_expanded_once(hip_ready):
    """A Q8_0 router imported read-only (ds3_hip_buffer_from_mmap, as the
    engine imports its mmap'd weights) is expanded to FP32 rows on its first
    call only; later calls read that copy.  Results are bit-equal to a
    writable import of the same bytes on the decode (T=1), certified batch
    (T=4) and grouped (T=64) paths.  Freeing the buffer drops the copy: a
    different router imported next, perhaps at the same address, routes by
    its own rows (oracle)."""
    spec = W.LayerSpec(ds3.TYPE_Q8_0, ds3.TYPE_Q8_0, ds3.TYPE_Q8_0, ds3.TYPE_Q8_0, n_embd=1024, n_ff=256,
                       n_expert=32)
    host = W.make_layer(spec, seed=4242)
    rw, ro = host.to_device(), host.to_device(readonly=True)
    one = np.zeros(1, np.uint8)
    assert hip().ds3_hip_buffer_write(ro.router, 0, one.ctypes.data, 1) == -1      # read-only
    for i, T in enumerate((1, 4, 64)):
        x = W.fill(W.NORMAL, 30 + T, T, T * spec.n_embd, 0.0, 1.0).reshape(T, spec.n_embd)
        print(f"  read-only Q8_0 router T={T}", flush=True)
        want, _ = _batch_run(rw, spec, x)
        got, ran = _batch_run(ro, spec, x)
        assert ("router_rows" in ran) == (i == 0)        # the copy is made by the first call only
        for a, b in zip(got, want):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # a second router, imported after the first is freed
    host2 = W.make_layer(spec, seed=4343)
    ro.router.close()
    ro2 = ds3.Buffer.from_mmap_array(host2.router)
    case2 = Case(spec, host=host2)
    x = W.fill(W.NORMAL, 99, 4, 4 * spec.n_embd, 0.0, 1.0).reshape(4, spec.n_embd)
    dev2 = W.DeviceLayer(spec=spec, router=ro2, experts=ro.experts)
    (got, gi, gs, _), ran = _batch_run(dev2, spec, x)
    assert "router_rows" in ran
    c1 = Case(spec, host=host)                           # the experts dev2 still uses
    case2.wg, case2.wu, case2.wd = c1.wg, c1.wu, c1.wd
    want, oi, osc, probs = case2.oracle(x)
    assert index_mismatches(gi, oi, probs) == 0
    assert_close(got, want)


def test_grouped_combine_unaligned_output(hip_ready):
    """The grouped path into output and residual rows that are not 16-byte
    aligned (views 4 bytes into their buffers): the combine then adds one
    column per thread instead of eight, with the same operations in the same
    order per column, so the result is the aligned call's, bit for bit."""
    spec = W.LayerSpec(n_embd=1024, n_ff=256, n_expert=128)
    case = Case(spec, seed=733)
    T, K = 100, spec.n_embd
    x = ds3.Buffer.from_array(W.fill(W.NORMAL, 19, T, T * K, 0.0, 1.0).reshape(T, K))
    base = np.full((T, K), 0.5, np.float32)
    resid = W.fill(W.NORMAL, 20, T, T * K, 0.0, 1.0).reshape(T, K)
    print(f"  grouped combine into unaligned rows, T={T}", flush=True)
    outs = []
    for off in (0, 4):
        ob = ds3.Buffer.alloc(T * K * 4 + 16)
        rb = ds3.Buffer.alloc(T * K * 4 + 16)
        out, res = ob.view(off, T * K * 4), rb.view(off, T * K * 4)
        out.write(base)
        res.write(resid)
        ds3.set_prefill_min_tokens(1)
        try:
            ds3.moe_ffn_batch(x, case.dev.router, spec.router_type, case.dev.experts, out, T, spec.n_expert,
                              W.N_USED, residual=res)
        finally:
            ds3.set_prefill_min_tokens(0)
        outs.append(out.read(np.float32, (T, K)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
