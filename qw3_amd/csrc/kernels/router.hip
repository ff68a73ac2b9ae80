// router.hip -- softmax + top-k + renormalisation, one wavefront per token.
//
// Semantics follow the reference oracle (src/ds3_reference.c:344-359 softmax,
// :466-490 top-k, :632-639 renorm): probabilities exp(l - max) / sum, k rounds
// of selection by (prob desc, index asc), then weights divided by their sum.
//
// Logits arrive either as one row per token or as nparts split-K partial
// rows (k_router_logits), summed here in a fixed order.
//
// Margin guard.  Router logits come from a parallel fp32 reduction, whose
// rounding differs from the reference's sequential sum.  To keep the selected
// experts (and their order) identical to the reference except for genuine
// ties, each token checks the gaps between its 9 largest logits against an
// error bound tau = 64 * 2^-24 * |x|_2 * max_e |W_e|_2.  If a gap is below
// 2*tau, every logit within 2*tau of the 9th is recomputed in the reference's
// order (i ascending, separate multiply and add roundings; the wave forms the
// exact products, one lane per candidate adds them in order), and selection
// runs on those values.  Logits further than 2*tau below the 9th cannot enter
// the top-k under either rounding, so they keep their fast values.
#include "common.h"
#include "launch.h"

namespace ds3k {

constexpr int ROUTE_MAX_E = 256;      // experts per token (4 per lane)
constexpr int ROUTE_EPL = ROUTE_MAX_E / WAVE;
constexpr int ROUTE_MAX_K = 32;
constexpr float GUARD_C = 64.0f;

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

// Element i of one router row as the reference's FP32 copy holds it
// (src/ds3_reference.c:87-184: the same products and roundings, no fusion).
template <int RT>
__device__ __forceinline__ float router_weight(const uint8_t *row, int i)
{
#pragma clang fp contract(off)
    if constexpr (RT == T_F32) {
        return ((const float *)row)[i];
    } else if constexpr (RT == T_F16) {
        return h2f(ld_u16(row + 2 * (size_t)i));
    } else if constexpr (RT == T_Q8_0) {
        const uint8_t *blk = row + (size_t)(i >> 5) * 34;
        return (float)(int8_t)blk[2 + (i & 31)] * h2f(ld_u16(blk));
    } else if constexpr (RT == T_Q4_K) {
        const uint8_t *blk = row + (size_t)(i >> 8) * 144;
        const int ib = i & 255, grp = ib >> 6, l = ib & 63;
        uint32_t sw[3];
#pragma unroll
        for (int w = 0; w < 3; w++)
            sw[w] = (uint32_t)blk[4 + 4 * w] | ((uint32_t)blk[5 + 4 * w] << 8) | ((uint32_t)blk[6 + 4 * w] << 16) |
                    ((uint32_t)blk[7 + 4 * w] << 24);
        float sc, mn;
        q4k_scale_min(sw[0], sw[1], sw[2], 2 * grp + (l >> 5), sc, mn);
        const int q = blk[16 + 32 * grp + (l & 31)];
        const float dl = h2f(ld_u16(blk)) * sc, ml = h2f(ld_u16(blk + 2)) * mn;
        return dl * (float)((l < 32) ? (q & 15) : (q >> 4)) - ml;
    } else {
        const uint8_t *blk = row + (size_t)(i >> 8) * 210;
        const int ib = i & 255, h = ib >> 7, t = (ib >> 5) & 3, l = ib & 31;
        const int qlb = blk[64 * h + l + 32 * (t & 1)];
        const int code = (((t < 2) ? (qlb & 15) : (qlb >> 4)) | (((blk[128 + 32 * h + l] >> (2 * t)) & 3) << 4)) - 32;
        const float sc = (float)(int8_t)blk[192 + 8 * h + (l >> 4) + 2 * t];
        return h2f(ld_u16(blk + 208)) * sc * (float)code;
    }
}

constexpr int GUARD_GROUP = 4;             // candidates recomputed together
constexpr int GUARD_PER_LANE = 8;          // k values per lane per pass
constexpr int GUARD_CHUNK = GUARD_PER_LANE * WAVE;
constexpr int GUARD_ROW = GUARD_CHUNK + 4; // LDS floats per candidate row (padded)

template <int RT>
__device__ __forceinline__ void guard_fetch(const float *x, int K, const uint8_t *const (&rows)[GUARD_GROUP], int nc,
                                            int k0, int lane, float (&xv)[GUARD_PER_LANE],
                                            float (&wv)[GUARD_GROUP][GUARD_PER_LANE])
{
    const int kb = k0 + GUARD_PER_LANE * lane;
#pragma unroll
    for (int i = 0; i < GUARD_PER_LANE; i++) xv[i] = kb + i < K ? x[kb + i] : 0.0f;
#pragma unroll
    for (int c = 0; c < GUARD_GROUP; c++)
#pragma unroll
        for (int i = 0; i < GUARD_PER_LANE; i++)
            wv[c][i] = (c < nc && kb + i < K) ? router_weight<RT>(rows[c], kb + i) : 0.0f;
}

// Reference-order dot products for up to GUARD_GROUP candidate experts of one
// token (src/ds3_reference.c:424-434: acc += x[i]*w[i], i ascending, product
// and sum rounded separately).  Per 512-wide chunk the wave forms the exact
// products of every candidate (lane l: k = 8l..8l+7) into LDS, issues the
// loads of the next chunk, and lane c adds candidate c's 512 products in
// index order (zero products past K change no sum).  Returns the logit in
// lane c < nc.
template <int RT>
__device__ float guard_recompute(const float *x, int K, const uint8_t *rw, uint64_t rstride, const int *cand, int nc,
                                 float *prod, int lane)
{
#pragma clang fp contract(off)
    const uint8_t *rows[GUARD_GROUP];
#pragma unroll
    for (int c = 0; c < GUARD_GROUP; c++) rows[c] = rw + (size_t)cand[c < nc ? c : 0] * rstride;
    float xv[GUARD_PER_LANE], wv[GUARD_GROUP][GUARD_PER_LANE];
    guard_fetch<RT>(x, K, rows, nc, 0, lane, xv, wv);
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += GUARD_CHUNK) {
#pragma unroll
        for (int c = 0; c < GUARD_GROUP; c++) {
            if (c < nc) {
                float pr[GUARD_PER_LANE];
#pragma unroll
                for (int i = 0; i < GUARD_PER_LANE; i++) pr[i] = xv[i] * wv[c][i];
                float4 *dst = (float4 *)(prod + c * GUARD_ROW + GUARD_PER_LANE * lane);
#pragma unroll
                for (int i = 0; i < GUARD_PER_LANE / 4; i++)
                    dst[i] = make_float4(pr[4 * i], pr[4 * i + 1], pr[4 * i + 2], pr[4 * i + 3]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (k0 + GUARD_CHUNK < K) guard_fetch<RT>(x, K, rows, nc, k0 + GUARD_CHUNK, lane, xv, wv);
        if (lane < nc) {
            const float4 *pr = (const float4 *)(prod + lane * GUARD_ROW);
#pragma unroll
            for (int b = 0; b < GUARD_CHUNK / 64; b++) {
                float4 v[16];
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = pr[16 * b + i];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    acc = acc + v[i].x;
                    acc = acc + v[i].y;
                    acc = acc + v[i].z;
                    acc = acc + v[i].w;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    return acc;
}

__device__ float guard_recompute_t(int rtype, const float *x, int K, const uint8_t *rw, uint64_t rstride,
                                   const int *cand, int nc, float *prod, int lane)
{
    switch (rtype) {
    case T_F32: return guard_recompute<T_F32>(x, K, rw, rstride, cand, nc, prod, lane);
    case T_F16: return guard_recompute<T_F16>(x, K, rw, rstride, cand, nc, prod, lane);
    case T_Q8_0: return guard_recompute<T_Q8_0>(x, K, rw, rstride, cand, nc, prod, lane);
    case T_Q4_K: return guard_recompute<T_Q4_K>(x, K, rw, rstride, cand, nc, prod, lane);
    default: return guard_recompute<T_Q6_K>(x, K, rw, rstride, cand, nc, prod, lane);
    }
}

// ---------------------------------------------------------------------------
// Router logits on fp32 MFMA (v_mfma_f32_16x16x4_f32), split over K.
// part[ks][t][e] = sum over k in chunk ks of x[t][k] * W[e][k].  A workgroup
// covers 32 tokens x all experts x one K chunk; wave w owns expert blocks
// w, w+4, ... of 16.  Per 16-wide K block, lane group g (lanes 16g..16g+15)
// holds k = 4g..4g+3 for both operands, one k per MFMA step, so A and B share
// the K order.  With blockIdx.x == 0 the kernel also writes the chunk's
// sum of W[e][k]^2 to wn[ks][e] (the guard's row norms).
// ---------------------------------------------------------------------------
typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr int RL_TOK = 32;
constexpr int RL_NBW = 4;                  // max expert blocks per wave (E <= 256)

__device__ __forceinline__ float4 router_w4(int rtype, const uint8_t *row, int k)
{
    if (rtype == T_F32) return *(const float4 *)((const float *)row + k);
    if (rtype == T_F16) {
        const uint2 h = *(const uint2 *)((const uint16_t *)row + k);
        return make_float4(h2f(h.x & 0xffffu), h2f(h.x >> 16), h2f(h.y & 0xffffu), h2f(h.y >> 16));
    }
    const uint8_t *blk = row + (size_t)(k >> 5) * 34;      // Q8_0, 4 values inside one block
    const float d = h2f(ld_u16(blk));
    const uint32_t q = ld_u32_a2(blk + 2 + (k & 31));
    return make_float4((float)(int8_t)byte_of(q, 0) * d, (float)(int8_t)byte_of(q, 1) * d,
                       (float)(int8_t)byte_of(q, 2) * d, (float)(int8_t)byte_of(q, 3) * d);
}

__global__ void __launch_bounds__(256)
k_router_logits(const float *__restrict__ x, int T, int K, int E, int rtype, const uint8_t *__restrict__ rw,
                uint64_t rstride, int kc, float *__restrict__ part, float *__restrict__ wmax,
                float *__restrict__ xsq, _Float16 *__restrict__ x16)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int t0 = blockIdx.x * RL_TOK;
    const int ks = blockIdx.y;
    const int kbeg = ks * kc;
    const int nbt = E / 16;
    const int mblocks = min(2, (T - t0 + 15) / 16);
    const bool want_norm = blockIdx.x == 0;

    floatx4 acc[2][RL_NBW];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < RL_NBW; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };
    float w2[RL_NBW] = { 0.f, 0.f, 0.f, 0.f };
    float x2[2] = { 0.f, 0.f };

    const float *xr[2];
#pragma unroll
    for (int mb = 0; mb < 2; mb++) {
        const int t = t0 + 16 * mb + r;
        xr[mb] = t < T ? x + (int64_t)t * K : nullptr;
    }
    // 64-wide K groups: every operand load of the group is issued before its
    // MFMAs (4 blocks of 16; lane group g takes k = 4g..4g+3 of each block)
    for (int kg = kbeg; kg < kbeg + kc; kg += 64) {
        float4 a[4][2], b[4][RL_NBW];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = kg + 16 * q + 4 * g;
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
                a[q][mb] = (mb < mblocks && xr[mb]) ? *(const float4 *)(xr[mb] + k) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int j = 0; j < RL_NBW; j++) {
                const int nb = wave + 4 * j;
                b[q][j] = nb < nbt ? router_w4(rtype, rw + (size_t)(16 * nb + r) * rstride, k)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        // by-products of the x tile: |x|^2 partials (wave 0) and the fp16
        // copy the grouped products read (wave w converts K block q = w)
#pragma unroll
        for (int q = 0; q < 4; q++) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const float4 v = a[q][mb];
                if (wave == 0) x2[mb] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                if (x16 != nullptr && wave == q && mb < mblocks && xr[mb]) {
                    half4_t h;
                    h[0] = (_Float16)v.x; h[1] = (_Float16)v.y; h[2] = (_Float16)v.z; h[3] = (_Float16)v.w;
                    *(half4_t *)(x16 + (int64_t)(t0 + 16 * mb + r) * K + kg + 16 * q + 4 * g) = h;
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
#pragma unroll
            for (int j = 0; j < RL_NBW; j++) {
                if (wave + 4 * j < nbt) {
                    const float4 bb = b[q][j];
                    if (want_norm) w2[j] += bb.x * bb.x + bb.y * bb.y + bb.z * bb.z + bb.w * bb.w;
#pragma unroll
                    for (int mb = 0; mb < 2; mb++) {
                        if (mb < mblocks) {
                            acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q][mb].x, bb.x, acc[mb][j], 0, 0, 0);
                            acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q][mb].y, bb.y, acc[mb][j], 0, 0, 0);
                            acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q][mb].z, bb.z, acc[mb][j], 0, 0, 0);
                            acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q][mb].w, bb.w, acc[mb][j], 0, 0, 0);
                        }
                    }
                }
            }
        }
    }
    float *pk = part + (int64_t)ks * T * E;
    float wm = 0.f;
#pragma unroll
    for (int j = 0; j < RL_NBW; j++) {
        const int nb = wave + 4 * j;
        if (nb >= nbt) continue;
#pragma unroll
        for (int mb = 0; mb < 2; mb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = t0 + 16 * mb + 4 * g + i;
                if (mb < mblocks && t < T) pk[(int64_t)t * E + 16 * nb + r] = acc[mb][j][i];
            }
        }
        if (want_norm) {
            float v = w2[j];
            v += __shfl_xor(v, 16, WAVE);
            v += __shfl_xor(v, 32, WAVE);
            wm = fmaxf(wm, v);
        }
    }
    if (wave == 0) {
#pragma unroll
        for (int mb = 0; mb < 2; mb++) {
            float v = x2[mb];
            v += __shfl_xor(v, 16, WAVE);
            v += __shfl_xor(v, 32, WAVE);
            const int t = t0 + 16 * mb + r;
            if (g == 0 && mb < mblocks && t < T) xsq[(int64_t)ks * T + t] = v;
        }
    }
    if (want_norm) {                            // uniform over the workgroup
        __shared__ float wm_s[4];
        wm = wave_max(wm);
        if (lane == 0) wm_s[wave] = wm;
        __syncthreads();
        if (threadIdx.x == 0) wmax[ks] = fmaxf(fmaxf(wm_s[0], wm_s[1]), fmaxf(wm_s[2], wm_s[3]));
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

__global__ void __launch_bounds__(256) k_route(RouteArgs a)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (t >= a.T) return;                      // whole wave leaves together
    const int E = a.E;
    const int wv = threadIdx.x / WAVE;
    const uint64_t below = (1ull << lane) - 1ull;
    __shared__ float prod_s[4][GUARD_GROUP * GUARD_ROW];
    __shared__ int cand_s[4][ROUTE_MAX_E];
    __shared__ float exact_s[4][ROUTE_MAX_E];

    // inputs of the error bound, loaded up front with the logits
    float ssp = 0.f, wmp = 0.f;
    if (a.x != nullptr) {
        if (a.xsq_parts)
            for (int p = lane; p < a.nparts; p += WAVE) ssp += a.xsq_parts[(int64_t)p * a.T + t];
        if (a.wmax_parts) {
            for (int p = lane; p < a.nparts; p += WAVE) wmp += a.wmax_parts[p];
        } else {
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++) {
                const int e = lane + WAVE * j;
                if (e < E) wmp = fmaxf(wmp, a.wn_rows[e]);
            }
        }
    }

    // logits: one row, or the sum of a.nparts split-K partial rows in order
    // (loads issued RP_BATCH partials at a time; +0 padding changes no sum)
    constexpr int RP_BATCH = 16;
    float l[ROUTE_EPL];
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) l[j] = 0.0f;
    const float *lg = a.logits + (int64_t)t * a.logit_stride;
    for (int p0 = 0; p0 < a.nparts; p0 += RP_BATCH) {
        float v[RP_BATCH][ROUTE_EPL];
#pragma unroll
        for (int u = 0; u < RP_BATCH; u++)
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++) {
                const int e = lane + WAVE * j;
                v[u][j] = (p0 + u < a.nparts && e < E) ? lg[(int64_t)(p0 + u) * a.part_stride + e] : 0.0f;
            }
#pragma unroll
        for (int u = 0; u < RP_BATCH; u++)
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++) l[j] += v[u][j];
    }
    bool finite = true;
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) {
        if (lane + WAVE * j >= E) l[j] = -INFINITY;
        else if (!__builtin_isfinite(l[j])) finite = false;
    }
    const bool all_finite = __all(finite);

    // Error bound tau = 64 * 2^-24 * |x|_2 * max_e |W_e|_2 (an upper bound on
    // the row norm: the sum of per-chunk maxima when the logits came in parts).
    const float *xt = a.x != nullptr ? a.x + (int64_t)t * a.K : nullptr;
    float tau = 0.f;
    if (a.x != nullptr) {
        if (!a.xsq_parts) {
            for (int i0 = 4 * lane; i0 < a.K; i0 += 4 * WAVE * 8) {
                float v[8][4];
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int k = i0 + 4 * WAVE * u + i;
                        v[u][i] = k < a.K ? xt[k] : 0.f;
                    }
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int i = 0; i < 4; i++) ssp += v[u][i] * v[u][i];
            }
        }
        const float ss = wave_sum(ssp);
        const float wmax = a.wmax_parts ? wave_sum(wmp) : wave_max(wmp);
        tau = GUARD_C * 0x1.0p-24f * sqrtf(ss) * sqrtf(wmax);
    }

    int32_t *oi = a.idx + (int64_t)t * a.out_stride;
    float *os = a.scores + (int64_t)t * a.out_stride;
    const int need = min(a.k + 1, E);

    // Fast path: the need = min(k+1, E) largest logits by a radix select on
    // order keys (ballot counts, no shuffles), ranked by (value desc, index
    // asc).  If every gap between neighbours exceeds both roundings (2 tau)
    // the reference ranks them the same way, and a gap above 2^-19 keeps
    // their probabilities at least 16 ulp apart, so expf cannot tie or
    // reorder them: the logit order is the reference's (prob desc) order.
    if (all_finite) {
        uint32_t key[ROUTE_EPL];
#pragma unroll
        for (int j = 0; j < ROUTE_EPL; j++) key[j] = lane + WAVE * j < E ? order_key(l[j]) : 0u;
        uint32_t thr = 0u;                      // largest key with >= need keys at or above it
        for (int bit = 31; bit >= 0; bit--) {
            const uint32_t tr = thr | (1u << bit);
            int cnt = 0;
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++) cnt += __popcll(__ballot(key[j] >= tr));
            if (cnt >= need) thr = tr;
        }
        int S = 0;
#pragma unroll
        for (int j = 0; j < ROUTE_EPL; j++) {
            const bool in = key[j] >= thr;
            const uint64_t m = __ballot(in);
            const int pos = S + __popcll(m & below);
            if (in && pos < WAVE) {
                cand_s[wv][pos] = lane + WAVE * j;
                exact_s[wv][pos] = l[j];
            }
            S += __popcll(m);
        }
        if (S <= WAVE) {                        // else: a tie wider than a wave, general path
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            float vi = 0.f;
            int ei = 0, rank = 0;
            if (lane < S) {
                vi = exact_s[wv][lane];
                ei = cand_s[wv][lane];
                for (int c = 0; c < S; c++) {
                    const float vc = exact_s[wv][c];
                    rank += (vc > vi || (vc == vi && cand_s[wv][c] < ei)) ? 1 : 0;
                }
            }
            float *ord_v = prod_s[wv];
            int *ord_e = (int *)(prod_s[wv] + WAVE);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            if (lane < S) {
                ord_v[rank] = vi;
                ord_e[rank] = ei;
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            const float my_v = lane < need ? ord_v[lane] : 0.f;
            const int my_e = lane < need ? ord_e[lane] : 0;
            const float prev_v = (lane >= 1 && lane < need) ? ord_v[lane - 1] : 0.f;
            const float gap_min = fmaxf(2.0f * tau, 0x1.0p-19f);
            const bool ok = lane == 0 || lane >= need || prev_v - my_v > gap_min;
            if (__all(ok)) {
                const float mx = ord_v[0];
                float sp = 0.f;
#pragma unroll
                for (int j = 0; j < ROUTE_EPL; j++)
                    if (lane + WAVE * j < E) sp += expf(l[j] - mx);
                const float inv = 1.0f / wave_sum(sp);
                const float p = expf(my_v - mx) * inv;
                float ssum = 0.f;
                for (int r = 0; r < a.k; r++) ssum += readlane_f(p, r);     // sequential, in k order
                if (a.logits_out) {
                    float *lo = a.logits_out + (int64_t)t * a.logit_stride;
#pragma unroll
                    for (int j = 0; j < ROUTE_EPL; j++) {
                        const int e = lane + WAVE * j;
                        if (e < E) lo[e] = l[j];
                    }
                }
                if (lane < a.k) {
                    float w = p;
                    if (a.norm && ssum > 0.0f) w *= 1.0f / ssum;
                    oi[lane] = my_e;
                    os[lane] = w;
                }
                return;                         // uniform over the wave
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
    }

    // General path: near ties (margin guard), non-finite logits, wide ties.
    if (a.x != nullptr && all_finite) {
        // the k-th largest logit (value desc, index asc)
        uint32_t taken = 0u;
        float kth = 0.f;
        for (int r = 0; r < a.k; r++) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++) {
                const int e = lane + WAVE * j;
                if (!((taken >> j) & 1u) && e < E && (l[j] > bv || (l[j] == bv && e < bi))) { bv = l[j]; bi = e; }
            }
            wave_argmax(bv, bi);
            if (bi < E && (bi & (WAVE - 1)) == lane) taken |= 1u << (bi / WAVE);
            kth = bv;
        }
        // Candidates: logits at least kth - 2*tau (nothing below can be
        // selected by the reference) that have another candidate within
        // 2*tau (only those can change rank); recompute them exactly.
        const float floor_v = kth - 2.0f * tau;
        int ns = 0;
#pragma unroll
        for (int j = 0; j < ROUTE_EPL; j++) {
            const int e = lane + WAVE * j;
            const bool in = e < E && l[j] >= floor_v;
            const uint64_t m = __ballot(in);
            if (in) {
                const int pos = ns + __popcll(m & below);
                cand_s[wv][pos] = e;
                exact_s[wv][pos] = l[j];
            }
            ns += __popcll(m);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        bool near[ROUTE_EPL];
        int my_e[ROUTE_EPL];
#pragma unroll
        for (int q = 0; q < ROUTE_EPL; q++) {
            const int i = lane + WAVE * q;
            near[q] = false;
            my_e[q] = -1;
            if (i < ns) {
                const float v = exact_s[wv][i];
                my_e[q] = cand_s[wv][i];
                for (int c = 0; c < ns; c++)
                    if (c != i && fabsf(exact_s[wv][c] - v) <= 2.0f * tau) near[q] = true;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        int nc = 0;                             // compact the near ones in place
#pragma unroll
        for (int q = 0; q < ROUTE_EPL; q++) {
            const uint64_t nm = __ballot(near[q]);
            if (near[q]) cand_s[wv][nc + __popcll(nm & below)] = my_e[q];
            nc += __popcll(nm);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        for (int c0 = 0; c0 < nc; c0 += GUARD_GROUP) {
            const int n = min(GUARD_GROUP, nc - c0);
            const float v = guard_recompute_t(a.rtype, xt, a.K, a.rw, a.rstride, &cand_s[wv][c0], n, prod_s[wv], lane);
            if (lane < n) exact_s[wv][c0 + lane] = v;
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        for (int c = 0; c < nc; c++) {
            const int e = cand_s[wv][c];
            if ((e & (WAVE - 1)) == lane) {
#pragma unroll
                for (int j = 0; j < ROUTE_EPL; j++)
                    if (j == e / WAVE) l[j] = exact_s[wv][c];
            }
        }
        if (lane == 0 && nc > 0 && a.guard_count) atomicAdd(a.guard_count, 1);
    }

    if (a.logits_out) {
        float *lo = a.logits_out + (int64_t)t * a.logit_stride;
#pragma unroll
        for (int j = 0; j < ROUTE_EPL; j++) {
            const int e = lane + WAVE * j;
            if (e < E) lo[e] = l[j];
        }
    }

    // Softmax.
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
    for (int r = 0; r < a.k; r++) {
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
    if (lane < a.k) {
        float w = sel_v;
        if (a.norm && ssum > 0.0f) w *= 1.0f / ssum;
        oi[lane] = sel_i;
        os[lane] = w;
    }
}

bool router_mfma_ok(int rtype, int K, int E, const void *x, const void *rw, uint64_t rstride)
{
    // float4 / 4-half loads of x rows and F32 / F16 router rows need 16 / 8-byte alignment
    if (((uintptr_t)x & 15) != 0) return false;
    if (rtype == T_F32 && ((((uintptr_t)rw) | rstride) & 15) != 0) return false;
    if (rtype == T_F16 && ((((uintptr_t)rw) | rstride) & 7) != 0) return false;
    if (rtype == T_Q8_0 && ((((uintptr_t)rw) | rstride) & 1) != 0) return false;
    return (rtype == T_F32 || rtype == T_F16 || rtype == T_Q8_0) && K % 64 == 0 && E % 16 == 0 && E <= 256;
}

int router_parts(int T, int K)
{
    const int tiles = (T + RL_TOK - 1) / RL_TOK;
    int ks = 256 / tiles;                      // ~256 workgroups
    if (ks < 1) ks = 1;
    if (ks > K / 64) ks = K / 64;
    if (ks > 32) ks = 32;
    while (ks > 1 && (K / 64) % ks != 0) ks--;  // equal chunks, multiples of 64
    return ks;
}

hipError_t launch_router_logits(const float *x, int T, int K, int E, int rtype, const uint8_t *rw, uint64_t rstride,
                                int nparts, float *part, float *wmax, float *xsq, _Float16 *x16, hipStream_t s)
{
    if (!router_mfma_ok(rtype, K, E, x, rw, rstride) || T <= 0 || nparts < 1 || (K / 64) % nparts != 0 ||
        (x16 != nullptr && ((uintptr_t)x16 & 7) != 0))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((T + RL_TOK - 1) / RL_TOK), (unsigned)nparts);
    hipLaunchKernelGGL(k_router_logits, grid, dim3(256), 0, s, x, T, K, E, rtype, rw, rstride, K / nparts, part,
                       wmax, xsq, x16);
    return hipGetLastError();
}

hipError_t launch_route(const RouteArgs &a, hipStream_t s)
{
    if (a.T <= 0 || a.E <= 0 || a.E > ROUTE_MAX_E || a.k <= 0 || a.k > ROUTE_MAX_K || a.k > a.E || a.nparts < 1)
        return hipErrorInvalidValue;
    if (a.x != nullptr && a.wmax_parts == nullptr && a.wn_rows == nullptr) return hipErrorInvalidValue;
    const int waves = 4;
    hipLaunchKernelGGL(k_route, dim3((unsigned)((a.T + waves - 1) / waves)), dim3(waves * WAVE), 0, s, a);
    return hipGetLastError();
}

}  // namespace ds3k
