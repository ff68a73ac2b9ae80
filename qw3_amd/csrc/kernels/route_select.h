// route_select.h -- per-token expert selection shared by the router
// kernels and the fused decode kernel.
//
// Softmax + top-k + renorm of one token by one wavefront (route_token_row),
// and the certified router's selection of a token group by one workgroup
// (cert_select_tokens).  Device code only; every function is inline so that
// each translation unit carries its own copy.
#pragma once
#include "common.h"
#include "launch.h"

namespace ds3k {

constexpr int ROUTE_MAX_E = 256;      // experts per token (4 per lane)
constexpr int ROUTE_EPL = ROUTE_MAX_E / WAVE;
constexpr int ROUTE_MAX_K = 32;

// Wave-wide argmax of (value desc, index asc).  Every lane gets the winner.
__device__ __forceinline__ void wave_argmax(float &v, int &i)
{
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, WAVE);
        const int oi = __shfl_xor(i, o, WAVE);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
}

// Order-preserving map of finite floats (and infinities) to unsigned keys.
__device__ __forceinline__ uint32_t order_key(float v)
{
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float readlane_f(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Wavefront max of unsigned values (lanes without a source read 0).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Inverse of order_key.
__device__ __forceinline__ float key_float(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Softmax + top-k + renorm of one token by one wave from its E logits at lg
// (E <= 256); writes the k indices to oi and weights to os.  The pointers
// may address global memory or LDS.
__device__ inline int route_token_row(const float *lg, int E, int k, bool norm, int32_t *oi, float *os, int lane)
{
    float l[ROUTE_EPL];
    bool finite = true;
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) {
        const int e = lane + WAVE * j;
        l[j] = e < E ? lg[e] : -INFINITY;
        if (e < E && !__builtin_isfinite(l[j])) finite = false;
    }
    const bool all_finite = __all(finite);

    // Fast path, in registers: k rounds of a wavefront max over 32-bit keys
    // (the logit's order key with its low 8 bits replaced by 255 - e, so each
    // round's winner is unique and carries its index).  The truncation can
    // only misorder logits within 256 ulps of each other, so the result is
    // accepted only if every gap is above 2^-19: between neighbours in the
    // top k (a misordered pair shows a negative gap somewhere between them),
    // and between the k-th and the largest logit not taken (full keys).  Such
    // gaps keep the probabilities at least 16 ulp apart, so expf cannot tie
    // or reorder them: the logit order is then the reference's (prob desc)
    // order.
    if (all_finite) {
        uint32_t key[ROUTE_EPL], full[ROUTE_EPL];
#pragma unroll
        for (int j = 0; j < ROUTE_EPL; j++) {
            const int e = lane + WAVE * j;
            full[j] = e < E ? order_key(l[j]) : 0u;             // finite logits: >= 2^23
            key[j] = e < E ? (full[j] & 0xffffff00u) | (uint32_t)(255 - e) : 0u;
        }
        int my_e = 0;
        float my_v = 0.f, prev_v = 0.f;
        for (int r = 0; r < k; r++) {
            uint32_t m = key[0];
#pragma unroll
            for (int j = 1; j < ROUTE_EPL; j++) m = max(m, key[j]);
            m = wave_max_u32(m);
            const int e = 255 - (int)(m & 255u);
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++)
                if (j == (e >> 6)) v = readlane_f(l[j], e & (WAVE - 1));
            my_e = lane == r ? e : my_e;
            my_v = lane == r ? v : my_v;
            prev_v = lane == r + 1 ? v : prev_v;
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++)
                if (lane + WAVE * j == e) {
                    key[j] = 0u;
                    full[j] = 0u;
                }
        }
        uint32_t rk = full[0];
#pragma unroll
        for (int j = 1; j < ROUTE_EPL; j++) rk = max(rk, full[j]);
        rk = wave_max_u32(rk);                                  // 0: no logit left
        bool ok = true;
        if (lane >= 1 && lane < k) ok = prev_v - my_v > 0x1.0p-19f;
        if (lane == k - 1 && rk != 0u) ok = ok && my_v - key_float(rk) > 0x1.0p-19f;
        if (__all(ok)) {
            const float mx = readlane_f(my_v, 0);
            float sp = 0.f;
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++)
                if (lane + WAVE * j < E) sp += expf(l[j] - mx);
            const float inv = 1.0f / wave_sum(sp);
            const float p = expf(my_v - mx) * inv;
            float ssum = 0.f;
            for (int r = 0; r < k; r++) ssum += readlane_f(p, r);     // sequential, in k order
            if (lane < k) {
                float w = p;
                if (norm && ssum > 0.0f) w *= 1.0f / ssum;
                oi[lane] = my_e;
                os[lane] = w;
            }
            return lane < k ? my_e : -1;        // uniform over the wave
        }
    }

    // General path: close logits, non-finite logits, wide ties.  Softmax.
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) mx = fmaxf(mx, l[j]);
    mx = wave_max(mx);
    float p[ROUTE_EPL];
    float sp = 0.f;
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) {
        const int e = lane + WAVE * j;
        p[j] = e < E ? expf(l[j] - mx) : 0.f;
        sp += p[j];
    }
    const float inv = 1.0f / wave_sum(sp);
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) p[j] *= inv;

    // Top-k by (prob desc, index asc).
    float sel_v = 0.f, ssum = 0.f;
    int sel_i = 0;
    for (int r = 0; r < k; r++) {
        float bv = -1.0f;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < ROUTE_EPL; j++) {
            const int e = lane + WAVE * j;
            // a NaN probability ranks below every number but stays selectable,
            // so each round always yields an index < E (k <= E)
            const float key = (p[j] == p[j]) ? p[j] : -0.5f;
            if (e < E && key > -1.5f && (key > bv || (key == bv && e < bi))) { bv = key; bi = e; }
        }
        wave_argmax(bv, bi);
        if ((bi & (WAVE - 1)) == lane) {                      // remove from later rounds
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++)
                if (j == bi / WAVE) p[j] = -2.0f;
        }
        ssum += bv;                                           // sequential, in k order
        if (lane == r) { sel_v = bv; sel_i = bi; }
    }
    if (lane < k) {
        float w = sel_v;
        if (norm && ssum > 0.0f) w *= 1.0f / ssum;
        oi[lane] = sel_i;
        os[lane] = w;
    }
    return lane < k ? sel_i : -1;
}

// Softmax + top-k + renorm of token t of a by one wave; lane r < k gets the
// expert of rank r back (the value it stored), the other lanes -1.
__device__ inline int route_token(const RouteArgs &a, int t, int lane)
{
    return route_token_row(a.logits + (int64_t)t * a.logit_stride, a.E, a.k, a.norm, a.idx + (int64_t)t * a.out_stride,
                    a.scores + (int64_t)t * a.out_stride, lane);
}

// ---------------------------------------------------------------------------
// Certified router (latency path for few tokens).
//
// The reference's logit is a chain of K dependent fp32 additions
// (src/ds3_reference.c:424-434): ~K * 6 cycles of latency however many lanes
// are free.  Instead, for each (token, expert):
//   S = sum_i p_i in fp64, where p_i = fl32(x_i * w_i) are the reference's
//       own rounded products (exact in fp64), and
//   B >= |reference logit - S|, a proven bound.  The reference's k-th partial
//       sum rounds once, |s^_k - (s^_{k-1} + p_k)| <= u |s^_k| (u = 2^-24), so
//       |s^_K - s_K| <= u sum_k |s^_k| <= u A / (1 - K u), A = sum_k |s_k|
//       over the exact prefix sums s_k of the p_i.  A is evaluated from the
//       same products (lane-local prefixes, a wavefront scan, the workgroup's
//       wave totals) and inflated by a bound on its own rounding; the host
//       folds every constant into bfac (router_cert_bfac):
//       B = bfac * A_computed + 1e-35.
// k_router_sums: one workgroup per (token group, expert), each of its 4
// waves sums a quarter of K, so one memory round trip brings every operand.
// k_router_select: one workgroup per token group ranks the experts by
// (fl32(S) desc, index asc), then certifies the top k: every adjacent pair
// in that order, and the k-th against every other expert, must be separated
// by more than B_a + B_b + tau, where tau covers the reference's softmax
// roundings (l - max, expf, the normalisation; src/ds3_reference.c:344-359)
// so that its probabilities order the same way, strictly.  A certified
// token's top k, in order, is the reference's, and its weights come from
// the fl32(S) logits.  A token that fails (about 2 % at N(0, 0.02) routers)
// is repaired: every expert that could still reach the top k gets the
// reference's exact sequential chain, then the ordinary selection runs on
// the repaired row.
// ---------------------------------------------------------------------------
constexpr int RC_WAVES = 4;
constexpr int RC_THREADS = 64 * RC_WAVES;

// DPP lane moves: row_shr:n inside rows of 16 lanes, row_bcast:15 / :31,
// wave_shr:1.  Lanes without a source lane read 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_d(double v)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROW_MASK, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROW_MASK, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Inclusive prefix sum over the wavefront: four row_shr steps inside each
// row of 16, then rows 1 and 3 add lane 15 of the row below, rows 2 and 3
// lane 31.  Every result is a tree of at most 6 additions.
__device__ __forceinline__ float wave_incl_scan(float v)
{
    v = v + dpp_f<0x111>(v);
    v = v + dpp_f<0x112>(v);
    v = v + dpp_f<0x114>(v);
    v = v + dpp_f<0x118>(v);
    v = v + dpp_f<0x142, 0xa>(v);
    v = v + dpp_f<0x143, 0xc>(v);
    return v;
}

__device__ __forceinline__ double wave_incl_scan_f64(double v)
{
    v = v + dpp_d<0x111>(v);
    v = v + dpp_d<0x112>(v);
    v = v + dpp_d<0x114>(v);
    v = v + dpp_d<0x118>(v);
    v = v + dpp_d<0x142, 0xa>(v);
    v = v + dpp_d<0x143, 0xc>(v);
    return v;
}

__device__ __forceinline__ double readlane_d(double v, int l)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Spacing of fp32 numbers at magnitude m: 2^(e - 23) for m in [2^e, 2^(e+1)).
__device__ __forceinline__ double f32_ulp(double m)
{
    const float f = (float)fmax(m, 1e-30);
    return (double)ldexpf(1.0f, ilogbf(f) - 23);
}

// Order-preserving unsigned key of a double (larger value, larger key).
__device__ __forceinline__ unsigned long long order_key_d(double v)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    return (u & 0x8000000000000000ull) ? ~u : (u | 0x8000000000000000ull);
}

// L contiguous floats at p (16-, 8- or 4-byte loads as L allows).
template <int L>
__device__ __forceinline__ void load_run(const float *p, float (&v)[L])
{
    if constexpr (L % 4 == 0) {
#pragma unroll
        for (int i = 0; i < L; i += 4) {
            const float4 q = *(const float4 *)(p + i);
            v[i] = q.x; v[i + 1] = q.y; v[i + 2] = q.z; v[i + 3] = q.w;
        }
    } else if constexpr (L % 2 == 0) {
#pragma unroll
        for (int i = 0; i < L; i += 2) {
            const float2 q = *(const float2 *)(p + i);
            v[i] = q.x; v[i + 1] = q.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < L; i++) v[i] = p[i];
    }
}

// Emit the k selected experts of a token from its fp32 logits (l: this
// lane's experts lane + 64 j) in the order given by (my_e, my_v) of lanes
// 0..k-1: the reference's softmax over all E logits, top-k values,
// renormalisation (src/ds3_reference.c:344-359, 632-639).
__device__ __forceinline__ void emit_ranked(const RouteArgs &a, int t, const float (&l)[ROUTE_EPL], float my_v,
                                            float mx, int my_e, int lane)
{
    const int E = a.E;
    float sp = 0.f;
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++)
        if (lane + WAVE * j < E) sp += expf(l[j] - mx);
    const float inv = 1.0f / wave_sum(sp);
    const float p = expf(my_v - mx) * inv;
    float ssum = 0.f;
    for (int r = 0; r < a.k; r++) ssum += readlane_f(p, r);     // sequential, in k order
    if (lane < a.k) {
        float wt = p;
        if (a.norm && ssum > 0.0f) wt *= 1.0f / ssum;
        a.idx[(int64_t)t * a.out_stride + lane] = my_e;
        a.scores[(int64_t)t * a.out_stride + lane] = wt;
    }
}

// Exact reference chains for the candidate experts of token t (the whole
// workgroup): the products of nb candidates at a time go to LDS, then lane m
// of wave 0 adds candidate m's in order and overwrites its logit.
__device__ inline void cert_repair(const float *__restrict__ x, int K, const float *__restrict__ w, int64_t wstride,
                            int t, const uint64_t (&cand)[4], float *logits_row, int nb, float *prod)
{
#pragma clang fp contract(off)
    __shared__ int list_s[ROUTE_MAX_E];
    __shared__ int n_s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    {
        const uint64_t m = cand[wave];
        int pre = 0;
        for (int j = 0; j < wave; j++) pre += __popcll(cand[j]);
        if ((m >> lane) & 1ull) list_s[pre + __popcll(m & ((1ull << lane) - 1ull))] = tid;
        if (tid == 0) n_s = __popcll(cand[0]) + __popcll(cand[1]) + __popcll(cand[2]) + __popcll(cand[3]);
    }
    __syncthreads();
    const int n = n_s;
    const int rowf = K + 4;
    const float *xr = x + (int64_t)t * K;
    for (int b0 = 0; b0 < n; b0 += nb) {
        const int nbb = min(nb, n - b0);
        for (int m = wave; m < nbb; m += RC_WAVES) {
            const float *wr = w + (int64_t)list_s[b0 + m] * wstride;
            for (int i = 4 * lane; i < K; i += 4 * WAVE) {
                const float4 wq = *(const float4 *)(wr + i), xq = *(const float4 *)(xr + i);
                float4 p;
                p.x = xq.x * wq.x;
                p.y = xq.y * wq.y;
                p.z = xq.z * wq.z;
                p.w = xq.w * wq.w;
                *(float4 *)(prod + (int64_t)m * rowf + i) = p;
            }
        }
        __syncthreads();
        if (tid < nbb) {
            const float *pr = prod + (int64_t)tid * rowf;
            float acc = 0.0f;
            for (int i = 0; i < K; i += 16) {
                float4 v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) v[q] = *(const float4 *)(pr + i + 4 * q);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    acc = acc + v[q].x;
                    acc = acc + v[q].y;
                    acc = acc + v[q].z;
                    acc = acc + v[q].w;
                }
            }
            logits_row[list_s[b0 + tid]] = acc;
        }
        __syncthreads();
    }
}

// DPP moves whose lanes without a source (and rows outside ROW_MASK) keep
// `old`: the identity of the reduction.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_fo(float v, float old)
{
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_do(double v, double old)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v), o = __builtin_bit_cast(uint64_t, old);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)o, (int)(uint32_t)b, CTRL, ROW_MASK,
                                                              0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(o >> 32), (int)(uint32_t)(b >> 32),
                                                              CTRL, ROW_MASK, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Wavefront max (the same scan pattern as wave_incl_scan; lane 63 holds it).
__device__ __forceinline__ float wave_max_dpp(float v)
{
    v = fmaxf(v, dpp_fo<0x111>(v, -INFINITY));
    v = fmaxf(v, dpp_fo<0x112>(v, -INFINITY));
    v = fmaxf(v, dpp_fo<0x114>(v, -INFINITY));
    v = fmaxf(v, dpp_fo<0x118>(v, -INFINITY));
    v = fmaxf(v, dpp_fo<0x142, 0xa>(v, -INFINITY));
    v = fmaxf(v, dpp_fo<0x143, 0xc>(v, -INFINITY));
    return readlane_f(v, 63);
}

__device__ __forceinline__ double wave_max_dpp_d(double v)
{
    v = fmax(v, dpp_do<0x111>(v, -INFINITY));
    v = fmax(v, dpp_do<0x112>(v, -INFINITY));
    v = fmax(v, dpp_do<0x114>(v, -INFINITY));
    v = fmax(v, dpp_do<0x118>(v, -INFINITY));
    v = fmax(v, dpp_do<0x142, 0xa>(v, -INFINITY));
    v = fmax(v, dpp_do<0x143, 0xc>(v, -INFINITY));
    return readlane_d(v, 63);
}

// Outputs of a certified token t from its ranking (lane r < k: expert
// e_rank of rank r; the fl32(S) logits): the reference's softmax over all E
// logits, the top-k values, renormalisation (src/ds3_reference.c:344-359,
// 632-639); writes idx / scores and counts the token.  One wavefront.
template <int EPL>
__device__ inline void cert_emit(const CertArgs &ca, const RouteArgs &a, int t, int lane, int e_rank)
{
    const int E = a.E, k = a.k;
    const double *Srow = ca.S + (int64_t)t * E;
    float lf[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) lf[j] = (float)Srow[min(lane + WAVE * j, E - 1)];
    const float my_v = (float)Srow[lane < k ? e_rank : 0];
    const float mx = readlane_f(my_v, 0);
    float sp = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; j++)
        if (lane + WAVE * j < E) sp += expf(lf[j] - mx);
    const float inv = 1.0f / readlane_f(wave_incl_scan(sp), 63);
    const float p = expf(my_v - mx) * inv;
    float ssum = 0.f;
    for (int r = 0; r < k; r++) ssum += readlane_f(p, r);     // sequential, in k order
    if (lane < k) {
        float wt = p;
        if (a.norm && ssum > 0.0f) wt *= 1.0f / ssum;
        a.idx[(int64_t)t * a.out_stride + lane] = e_rank;
        a.scores[(int64_t)t * a.out_stride + lane] = wt;
    }
    if (lane == 0 && ca.stats != nullptr) atomicAdd(&ca.stats[0], 1ull);
}

__device__ inline void cert_emit_any(const CertArgs &ca, const RouteArgs &a, int t, int lane, int e_rank)
{
    switch ((a.E + WAVE - 1) / WAVE) {                // uniform
    case 1: cert_emit<1>(ca, a, t, lane, e_rank); break;
    case 2: cert_emit<2>(ca, a, t, lane, e_rank); break;
    case 3: cert_emit<3>(ca, a, t, lane, e_rank); break;
    default: cert_emit<4>(ca, a, t, lane, e_rank); break;
    }
}

// The certified selection of token t by one wavefront, in registers: no
// workgroup barrier, no LDS -- the common case of cert_select_tokens.  Lane
// l holds experts l + 64 j (EPL of them).  k rounds of a wavefront max over
// 32-bit keys (the order key of fl32(S) with its low 8 bits replaced by
// 255 - e) give the top k in order with no search for the winner; the
// truncation can only put experts within 256 ulps of each other out of
// order, and any such pair fails the certification test below (their bounds
// overlap by far more), which is that of cert_select_tokens.  Returns
// whether the token is certified (wave-uniform); if so, lane r < k gets the
// expert of rank r in e_rank and, with emit, the token's idx / scores are
// written and counted.  A token with a non-finite value, or one that fails
// the test, returns false and is left to cert_select_tokens.
template <int EPL>
__device__ inline bool cert_select_wave_e(const CertArgs &ca, const RouteArgs &a, int t, bool emit, int lane,
                                          int &e_rank)
{
    const int E = a.E, k = a.k;
    const double *Srow = ca.S + (int64_t)t * E;
    const float *Brow = ca.B + (int64_t)t * E;
    double s[EPL];
    float b[EPL], lf[EPL];
    uint32_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) {                   // every load issued before any use
        const int e = min(lane + WAVE * j, E - 1);
        s[j] = Srow[e];
        b[j] = Brow[e];
    }
    bool fin = true;
    uint32_t sm = 0u, bm = 0u;                        // max |fl32(S)| and max B as bit patterns (both >= 0)
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = lane + WAVE * j;
        const bool v = e < E;
        lf[j] = (float)s[j];
        if (v && (!__builtin_isfinite(s[j]) || !__builtin_isfinite(b[j]) || !__builtin_isfinite(lf[j]))) fin = false;
        key[j] = v ? (order_key(lf[j]) & 0xffffff00u) | (uint32_t)(255 - e) : 0u;   // > 0 when present
        sm = max(sm, v ? __float_as_uint(fabsf(lf[j])) : 0u);
        bm = max(bm, v ? __float_as_uint(b[j]) : 0u);
    }
    if (!__all(fin)) return false;
    // k rounds: the largest remaining key; rank r's expert goes to lane r, its successor's to lane r - 1
    int my_e = 0, nx_e = 0;
    for (int r = 0; r < k; r++) {
        uint32_t m = key[0];
#pragma unroll
        for (int j = 1; j < EPL; j++) m = max(m, key[j]);
        m = wave_max_u32(m);
        const int e = 255 - (int)(m & 255u);
        my_e = lane == r ? e : my_e;
        nx_e = lane + 1 == r ? e : nx_e;
#pragma unroll
        for (int j = 0; j < EPL; j++)
            if (lane + WAVE * j == e) key[j] = 0u;
    }
    const int le = lane < k ? my_e : 0, ln = lane + 1 < k ? nx_e : 0;
    const double my_s = Srow[le], nx_s = Srow[ln];      // cached: read a moment ago
    const float my_b = Brow[le], nx_b = Brow[ln];
    // the best of the rest: max of S + B over the experts not taken
    double hv = -INFINITY;
#pragma unroll
    for (int j = 0; j < EPL; j++)
        if (key[j] != 0u) hv = fmax(hv, s[j] + (double)b[j]);
    const double hi = wave_max_dpp_d(hv);
    const double bmax = (double)__uint_as_float(wave_max_u32(bm));
    const double ulp2 = 2.0 * f32_ulp((double)__uint_as_float(wave_max_u32(sm)));
    const double s_top = readlane_d(my_s, 0), b_top = (double)readlane_f(my_b, 0);
    bool ok = true;
    if (lane < k) {
        double lo, sb;
        if (lane + 1 < k) {
            sb = nx_s;
            lo = nx_s + (double)nx_b;
        } else {
            sb = hi;
            lo = hi;
        }
        const double span = (sb > -INFINITY ? s_top - sb : 0.0) + b_top + bmax;
        const double tau = 0x1.0p-18 + ulp2 + 0x1.0p-23 * span;
        ok = my_s - (double)my_b > lo + tau && s_top - my_s < 64.0;
    }
    if (!__all(ok)) return false;
    e_rank = my_e;
    if (emit) cert_emit<EPL>(ca, a, t, lane, my_e);
    return true;
}

__device__ inline bool cert_select_wave(const CertArgs &ca, const RouteArgs &a, int t, bool emit, int lane,
                                        int &e_rank)
{
    switch ((a.E + WAVE - 1) / WAVE) {                // uniform
    case 1: return cert_select_wave_e<1>(ca, a, t, emit, lane, e_rank);
    case 2: return cert_select_wave_e<2>(ca, a, t, emit, lane, e_rank);
    case 3: return cert_select_wave_e<3>(ca, a, t, emit, lane, e_rank);
    default: return cert_select_wave_e<4>(ca, a, t, emit, lane, e_rank);
    }
}

// ---------------------------------------------------------------------------
// Exact weights of a routed token.  A certified token's top k is the
// reference's, but fl32(S) is not its logit: the reference's chain rounds
// ~K times and lands up to B away, and the softmax carries that into the
// weights (~1e-5 relative at |logit| ~ 10).  So the selected experts' logits
// are recomputed as the reference's exact chains and the weights derived
// from them, off the critical path: a workgroup appended to the decode
// gate/up grid does it while the other workgroups stream the expert rows.
// ---------------------------------------------------------------------------

// One chain step for block (wq, xq) (elements 32 b + 4 j + c of lane 8 m + j):
// lane 8 m adds, in order, the four products of each lane 8 m + JJ, JJ =
// 0 .. 7, taking them through DPP row_shl:JJ (lane 8 m and 8 m + 7 share a
// row of 16 lanes).
template <int JJ>
__device__ __forceinline__ float chain_from_lane(float acc, const float (&q)[4])
{
#pragma clang fp contract(off)
    if constexpr (JJ == 0) {
        acc = acc + q[0];
        acc = acc + q[1];
        acc = acc + q[2];
        acc = acc + q[3];
    } else {
        acc = acc + dpp_f<0x100 + JJ>(q[0]);
        acc = acc + dpp_f<0x100 + JJ>(q[1]);
        acc = acc + dpp_f<0x100 + JJ>(q[2]);
        acc = acc + dpp_f<0x100 + JJ>(q[3]);
    }
    return acc;
}

__device__ __forceinline__ float chain_block(float acc, const float4 &wq, const float4 &xq)
{
#pragma clang fp contract(off)
    const float q[4] = { xq.x * wq.x, xq.y * wq.y, xq.z * wq.z, xq.w * wq.w };   // the reference's rounded products
    acc = chain_from_lane<0>(acc, q);
    acc = chain_from_lane<1>(acc, q);
    acc = chain_from_lane<2>(acc, q);
    acc = chain_from_lane<3>(acc, q);
    acc = chain_from_lane<4>(acc, q);
    acc = chain_from_lane<5>(acc, q);
    acc = chain_from_lane<6>(acc, q);
    return chain_from_lane<7>(acc, q);
}

// The exact chain is 2048 dependent fp32 additions per logit at K = 2048:
// ~4.5 cycles each, and any other instruction of the adding wave costs its
// issue slot on top (a DPP operand also stalls a dependent add by 2 wait
// states).  So the work is split: waves 1-3 (producers) stream the router
// rows of the selected experts into LDS by DMA, multiply them by the token's
// row and write the products transposed, block by block (a block = 32
// consecutive elements of each of 8 experts); lanes 0-7 of wave 0 (the
// consumer, lane m = expert m) read each expert's products in order and add
// them, their LDS reads issued three half-blocks ahead of the adds.  One
// workgroup barrier per chunk of XC_CH blocks hands a product buffer over.
// Measured on MI355X (per-chunk timestamps): ~7.5 cycles per add at 2.4 GHz
// whether the reads run one, two or three half-blocks ahead and with or
// without the row workgroups beside it, against 4.4 for a chain of adds on
// register operands alone.
#ifndef DS3_XC_CH
#define DS3_XC_CH 8
#endif
#ifndef DS3_XC_RP
#define DS3_XC_RP 7
#endif
constexpr int XC_CH = DS3_XC_CH;        // blocks per chunk
constexpr int XC_PS = 36;       // floats per expert in a block's products: 32 + 4 (conflict-free reads)
// LDS byte offset of half-block hb (16 products) of one expert's products
// within a chunk's product buffer.
__host__ __device__ constexpr uint32_t xc_half_off(int hb)
{
    return (uint32_t)((hb >> 1) * 8 * XC_PS * 4 + (hb & 1) * 64);
}
constexpr int XC_NP = 3;        // producer waves
constexpr int XC_RP = DS3_XC_RP;        // DMA ring slots (1 KiB blocks) per producer wave: ~1.4 us of lookahead
constexpr int XC_THREADS = (XC_NP + 1) * WAVE;

// LDS of the exact stage: the token's row (K floats), two product buffers,
// the producers' DMA rings.
__host__ __device__ constexpr size_t exact_chain_lds(int K)
{
    return (size_t)K * 4 + (size_t)2 * XC_CH * 8 * XC_PS * 4 + (size_t)XC_NP * XC_RP * 1024;
}

// One 16-byte DMA per lane from src into LDS at lds_base + 16 * lane
// (global_load_lds_dwordx4, LDS base in M0, which the statement restores).
// Issued outside the compiler's view, so that it neither waits for the ring
// before every LDS access nor counts it: the caller's explicit vmcnt waits
// order it.  With WAIT it first waits for this wave's earlier LDS operations
// (a slot is rewritten only after it was read); without, the caller has
// already consumed every read of the slot (so the compiler waited for them).
template <bool WAIT = true>
__device__ __forceinline__ void chain_dma(const float *src, uint32_t lds_base)
{
    uint32_t m0_save;
    if constexpr (WAIT) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %2\n\t"
                 "global_load_lds_dwordx4 %1, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(m0_save)
                 : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_base))   // wave-uniform: in an SGPR
                 : "memory");
}

// The token's row into LDS (lds[0 .. K), K <= 4096) by the XC_THREADS
// threads of the workgroup, in two steps, so that other loads (the
// selection's) can be in flight between them.
__device__ __forceinline__ void exact_load_x(const float *__restrict__ xrow, int K, float4 (&xv)[4], int tid)
{
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int i = 4 * (tid + XC_THREADS * q);
        if (i < K) xv[q] = *(const float4 *)(xrow + i);
    }
}

__device__ __forceinline__ void exact_store_x(float *lds, int K, const float4 (&xv)[4], int tid)
{
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int i = 4 * (tid + XC_THREADS * q);
        if (i < K) *(float4 *)(lds + i) = xv[q];
    }
}

// Half a block of a chain's products (4 x 16 bytes at LDS byte address a)
// into d, read outside the compiler's scheduling: the consumer issues its
// reads ahead of its adds, and xc_wait_half<N> (N = the reads issued after
// them) waits for exactly those registers.
typedef float xc_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void xc_read_half(xc_f4 (&d)[4], uint32_t a)
{
#pragma unroll
    for (int i = 0; i < 4; i++) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d[i]) : "v"(a), "i"(16 * i));
}

template <int N>
__device__ __forceinline__ void xc_wait_half(xc_f4 (&d)[4])
{
    static_assert(N >= 0 && N <= 15, "lgkmcnt field holds 0..15");
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]) : "n"(N));
}

// The reference's logits of the experts in lanes 0 .. k-1 of e_lane (every
// wave holds them), exactly: acc = acc + x_i * w_i, i ascending, every
// product and sum rounded to fp32 (src/ds3_reference.c:424-434).  Called by
// all XC_THREADS threads of the workgroup (barriers inside) with the token's
// row staged at lds[0 .. K) and visible; lds: exact_chain_lds(K) bytes.
// Producer wave pw (wave pw + 1) owns blocks pw, pw + 3, ... and keeps XC_RP
// of them in flight.  8 experts per pass (lane 8 m + j of a producer
// multiplies elements 32 b + 4 j .. + 3 of expert m).  Wave 0, lane r < k,
// returns e_r's logit.  K % 256 == 0.
__device__ inline float exact_chain_wg(float *lds, int K, const float *__restrict__ w, int64_t wstride, int e_lane,
                                       int k, int wave, int lane)
{
#pragma clang fp contract(off)
    typedef __attribute__((address_space(3))) void lds_void;
    const float *xs = lds;
    float *pb = lds + K;                                    // [2][XC_CH][8][XC_PS]
    const int nb = K / 32, nch = nb / XC_CH, m = lane >> 3, j = lane & 7, pw = wave - 1;
    const float *wring = pb + 2 * XC_CH * 8 * XC_PS + max(pw, 0) * XC_RP * 256;   // this producer's DMA ring
    const uint32_t ring = (uint32_t)(uintptr_t)(lds_void *)wring;
    float res = 0.f;
    for (int p0 = 0; p0 < k; p0 += 8) {
        const float *wr = nullptr;
        int slot = 0;
        if (wave > 0) {
            const int e = __shfl(e_lane, min(p0 + m, k - 1), WAVE);
            wr = w + (int64_t)e * wstride + 4 * j;
            for (int q = 0; q < XC_RP; q++) chain_dma(wr + 32 * min(pw + XC_NP * q, nb - 1), ring + 1024u * q);
        }
        float acc = 0.f;
        for (int c = -1; c < nch; c++) {
            if (wave > 0) {
                const int cp = c + 1;                           // the chunk this round produces
                if (cp < nch) {
                    for (int b = cp * XC_CH; b < cp * XC_CH + XC_CH; b++) {
                        if (b % XC_NP != pw) continue;          // uniform over the wave
                        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(XC_RP - 1) : "memory");   // block b landed
                        const float4 wq = *(const float4 *)(wring + 256 * slot + 4 * lane);
                        const float4 xq = *(const float4 *)(xs + 32 * b + 4 * j);
                        const float4 pq = make_float4(xq.x * wq.x, xq.y * wq.y, xq.z * wq.z, xq.w * wq.w);
                        *(float4 *)(pb + (((cp & 1) * XC_CH + b % XC_CH) * 8 + m) * XC_PS + 4 * j) = pq;
                        // the slot's read fed the multiply above: no wait before the refill
                        chain_dma<false>(wr + 32 * min(b + XC_NP * XC_RP, nb - 1), ring + 1024u * slot);   // past the end: unused
                        slot = slot + 1 == XC_RP ? 0 : slot + 1;
                    }
                }
            } else if (c >= 0 && lane < 8) {
                // lane m adds expert m's products; the other lanes stay off,
                // so each LDS read returns 8 lanes' data instead of 64
                // block bb + 1's products are read while block bb's are added
                const uint32_t pc =
                    (uint32_t)(uintptr_t)(lds_void *)(pb + ((c & 1) * XC_CH * 8 + lane) * XC_PS);
                // Reads run three half-blocks (16 products each) ahead of
                // the adds: one block's reads take longer to return than its
                // 32 adds, and lgkmcnt counts at most 15 reads in flight.
                constexpr int NH = 2 * XC_CH;
                xc_f4 v[4][4];
#pragma unroll
                for (int hb = 0; hb < 3; hb++) xc_read_half(v[hb], pc + xc_half_off(hb));
#pragma unroll
                for (int hb = 0; hb < NH; hb++) {
                    if (hb + 3 < NH) {
                        xc_read_half(v[(hb + 3) % 4], pc + xc_half_off(hb + 3));
                        xc_wait_half<12>(v[hb % 4]);
                    } else if (hb + 2 < NH) {
                        xc_wait_half<8>(v[hb % 4]);
                    } else if (hb + 1 < NH) {
                        xc_wait_half<4>(v[hb % 4]);
                    } else {
                        xc_wait_half<0>(v[hb % 4]);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc = acc + v[hb % 4][i].x;
                        acc = acc + v[hb % 4][i].y;
                        acc = acc + v[hb % 4][i].z;
                        acc = acc + v[hb % 4][i].w;
                    }
                }
            }
            __syncthreads();                                    // chunk c consumed, chunk c + 1 written
        }
        if (wave > 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the ring drains before the next pass
        const float v = __shfl(acc, min(max(lane - p0, 0), 7), WAVE);
        if (lane >= p0 && lane < p0 + 8) res = v;
    }
    return res;
}

// Token t's routing outputs from the exact logits of its selected experts
// (every wave: lane r < k of e_lane = the expert of rank r, already the
// reference's order): the logits row supplies the other experts' values
// (fl32(S), or exact chains where a repair computed them), the selected
// entries are overwritten with their exact logits, and emit_ranked writes
// idx / scores (wave 0).  All XC_THREADS threads of the workgroup call it,
// with the token's row staged at lds[0 .. K) and visible.
__device__ inline void exact_weights_wg(float *lds, int K, const float *__restrict__ w, int64_t wstride,
                                        const RouteArgs &a, int t, int e_lane, int wave, int lane)
{
    float *lrow = (float *)a.logits + (int64_t)t * a.logit_stride;
    float l[ROUTE_EPL];
    if (wave == 0) {
#pragma unroll
        for (int jj = 0; jj < ROUTE_EPL; jj++) {            // lands during the chain
            const int e = lane + WAVE * jj;
            l[jj] = e < a.E ? lrow[e] : -INFINITY;
        }
    }
    const float v = exact_chain_wg(lds, K, w, wstride, e_lane, a.k, wave, lane);
    if (wave != 0) return;
    for (int r = 0; r < a.k; r++) {
        const int er = __builtin_amdgcn_readlane(e_lane, r);
        const float vr = readlane_f(v, r);
#pragma unroll
        for (int jj = 0; jj < ROUTE_EPL; jj++)
            if (lane + WAVE * jj == er) l[jj] = vr;
    }
    if (lane < a.k) lrow[e_lane] = v;
    emit_ranked(a, t, l, lane < a.k ? v : 0.f, readlane_f(v, 0), e_lane, lane);
}

// Rank, certify and, where needed, repair the routing of tokens t0 ..
// t0 + TG - 1 with the whole workgroup (RC_THREADS threads, all of which call
// it).  Returns the LDS array [TG][WAVE] whose entries 0 .. k-1 of row tt are
// the experts of token t0 + tt in the reference's order.  With emit it also
// writes the token's idx / scores (and repaired logits) through a and counts
// ca.stats; without, it writes LDS only, so any number of workgroups may
// route the same tokens.  prod: ca.nb LDS rows of K + 4 floats.
template <int TG>
__device__ inline const int *cert_select_tokens(const float *__restrict__ x, int K, const float *__restrict__ w,
                                                int64_t wstride, const CertArgs &ca, const RouteArgs &a, int t0,
                                                bool emit, float *prod)
{
    __shared__ double sS[TG][ROUTE_MAX_E];
    __shared__ float sB[TG][ROUTE_MAX_E];
    __shared__ __attribute__((aligned(16))) unsigned long long key_s[TG][ROUTE_MAX_E];
    __shared__ int rank_s[TG][ROUTE_MAX_E];
    __shared__ uint8_t sel_s[TG][ROUTE_MAX_E];
    __shared__ int ord_s[TG][WAVE];
    __shared__ float lg_s[TG][ROUTE_MAX_E];     // logits; exact chains for repaired candidates
    __shared__ float wt_s[TG][WAVE];
    __shared__ unsigned int bmax_s[TG];
    __shared__ unsigned long long smax_s[TG], hi_s[TG];
    __shared__ int bad_s[TG], fail_s[TG];
    __shared__ uint64_t cand_s[TG][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, k = a.k, T = a.T;
    constexpr int PER = (TG * ROUTE_MAX_E + RC_THREADS - 1) / RC_THREADS;
    const int E32 = (E + 31) & ~31;             // key rows padded with zero keys (below every expert)
    if (tid < TG) {
        bmax_s[tid] = 0u;
        smax_s[tid] = 0ull;
        hi_s[tid] = 0ull;                   // below every key: no other expert
        bad_s[tid] = 0;
        fail_s[tid] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int p = tid + RC_THREADS * r, tt = p / E, e = p - tt * E;
        if (tt >= TG || t0 + tt >= T) continue;
        const double s = ca.S[(int64_t)(t0 + tt) * E + e];
        const float b = ca.B[(int64_t)(t0 + tt) * E + e];
        const float lf = (float)s;
        sS[tt][e] = s;
        sB[tt][e] = b;
        lg_s[tt][e] = lf;
        sel_s[tt][e] = 0;
        rank_s[tt][e] = 0;
        key_s[tt][e] = ((unsigned long long)order_key(lf) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)e);
        if (!__builtin_isfinite(s) || !__builtin_isfinite(b) || !__builtin_isfinite(lf)) bad_s[tt] = 1;
        atomicMax(&bmax_s[tt], __float_as_uint(b));
        atomicMax(&smax_s[tt], __builtin_bit_cast(unsigned long long, fabs(s)));
    }
    __syncthreads();
    if (E32 > E)
        for (int q = tid; q < TG * (E32 - E); q += RC_THREADS) key_s[q / (E32 - E)][E + q % (E32 - E)] = 0ull;
    __syncthreads();
    // rank by (fl32(S) desc, index asc): the number of larger keys, counted
    // by `sub` threads per (token, expert) over E32 / sub keys each, 8 keys
    // (four 16-byte LDS reads) at a time
    {
        int sub = 1;
        while (sub < 4 && TG * E * sub * 2 <= RC_THREADS) sub *= 2;
        const int span = E32 / sub;
        for (int q = tid; q < TG * E * sub; q += RC_THREADS) {
            const int pr = q / sub, part = q - pr * sub, tt = pr / E, e = pr - tt * E;
            if (t0 + tt >= T) continue;
            const unsigned long long my = key_s[tt][e];
            int cnt = 0;
            for (int c = part * span; c < (part + 1) * span; c += 8) {
                const ulonglong2 *kp = (const ulonglong2 *)&key_s[tt][c];
                ulonglong2 v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = kp[i];
#pragma unroll
                for (int i = 0; i < 4; i++) cnt += (v[i].x > my ? 1 : 0) + (v[i].y > my ? 1 : 0);
            }
            atomicAdd(&rank_s[tt][e], cnt);
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int p = tid + RC_THREADS * r, tt = p / E, e = p - tt * E;
        if (tt >= TG || t0 + tt >= T) continue;
        const int rank = rank_s[tt][e];
        if (rank < k) {
            ord_s[tt][rank] = e;
            sel_s[tt][e] = 1;
        } else {
            atomicMax(&hi_s[tt], order_key_d(sS[tt][e] + (double)sB[tt][e]));
        }
    }
    __syncthreads();
    if (wave < TG && t0 + wave < T) {
        const int tt = wave, t = t0 + tt;
        const double bmax = (double)__uint_as_float(bmax_s[tt]);
        const double ulp2 = 2.0 * f32_ulp(__builtin_bit_cast(double, smax_s[tt]));
        const unsigned long long hk = hi_s[tt];
        const double hi = hk == 0ull ? -INFINITY
                                     : __builtin_bit_cast(double, (hk & 0x8000000000000000ull) ? (hk & ~0x8000000000000000ull)
                                                                                               : ~hk);
        const int e_top = ord_s[tt][0];
        const double s_top = sS[tt][e_top], b_top = sB[tt][e_top];
        bool ok = !bad_s[tt];
        double tau_k = 0.0;
        int my_e = 0;
        if (lane < k) {
            my_e = ord_s[tt][lane];
            const double sa = sS[tt][my_e], ba = sB[tt][my_e];
            double lo, sb;
            if (lane + 1 < k) {
                const int eb = ord_s[tt][lane + 1];
                sb = sS[tt][eb];
                lo = sb + (double)sB[tt][eb];
            } else {
                sb = hi;
                lo = hi;
            }
            const double span = (sb > -INFINITY ? s_top - sb : 0.0) + b_top + bmax;
            const double tau = 0x1.0p-18 + ulp2 + 0x1.0p-23 * span;
            // strictly separated, and the reference's expf of l - max stays normal
            ok = ok && sa - ba > lo + tau && s_top - sa < 64.0;
            if (lane + 1 == k) tau_k = tau;
        }
        const bool certified = __all(ok);
        if (emit && lane == 0 && ca.stats != nullptr) atomicAdd(&ca.stats[certified ? 0 : 1], 1ull);
        float l[ROUTE_EPL];
#pragma unroll
        for (int j = 0; j < ROUTE_EPL; j++) {
            const int e = lane + WAVE * j;
            l[j] = e < E ? (float)sS[tt][e] : -INFINITY;
        }
        if (certified) {
            if (emit) emit_ranked(a, t, l, lane < k ? (float)sS[tt][my_e] : 0.f, (float)s_top, my_e, lane);
        } else {
            // candidates: the top k, and every expert whose interval reaches
            // the k-th's (all experts when some value is not finite)
            tau_k = readlane_d(tau_k, k - 1);
            const double thr = sS[tt][ord_s[tt][k - 1]] - bmax - ulp2 - tau_k - 0x1.0p-18;
            const bool all = bad_s[tt] != 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = lane + WAVE * j;
                const bool in = e < E && (all || sel_s[tt][e] || sS[tt][e] + (double)sB[tt][e] >= thr);
                const uint64_t m = __ballot(in);
                if (lane == 0) cand_s[tt][j] = m;
            }
            if (lane == 0) fail_s[tt] = 1;
        }
    }
    __syncthreads();
    bool any = false;
    for (int tt = 0; tt < TG; tt++) {
        if (!fail_s[tt]) continue;                          // uniform over the workgroup
        any = true;
        const uint64_t cand[4] = { cand_s[tt][0], cand_s[tt][1], cand_s[tt][2], cand_s[tt][3] };
        cert_repair(x, K, w, wstride, t0 + tt, cand, lg_s[tt], ca.nb, prod);
    }
    if (any) {
        if (wave < TG && fail_s[wave]) {
            const int t = t0 + wave;
            route_token_row(lg_s[wave], E, k, a.norm, ord_s[wave], wt_s[wave], lane);
            if (emit) {
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                if (lane < k) {
                    a.idx[(int64_t)t * a.out_stride + lane] = ord_s[wave][lane];
                    a.scores[(int64_t)t * a.out_stride + lane] = wt_s[wave][lane];
                }
                float *lrow = (float *)a.logits + (int64_t)t * a.logit_stride;
                for (int e = lane; e < E; e += WAVE) lrow[e] = lg_s[wave][e];
            }
        }
        __syncthreads();
    }
    return &ord_s[0][0];
}

}  // namespace ds3k
