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

// Row value w(e, i) of the router matrix as the reference's FP32 copy holds it.
__device__ __forceinline__ float router_weight(int rtype, const uint8_t *rw, uint64_t rstride, int e, int i)
{
    const uint8_t *row = rw + (size_t)e * rstride;
    if (rtype == T_F32) return ((const float *)row)[i];
    if (rtype == T_F16) return h2f(((const uint16_t *)row)[i]);
    // Q8_0: exact product q * d
    const uint8_t *blk = row + (size_t)(i >> 5) * 34;
    const float d = h2f(ld_u16(blk));
    return (float)(int8_t)blk[2 + (i & 31)] * d;
}

constexpr int GUARD_GROUP = 8;             // candidates recomputed together
constexpr int GUARD_CHUNK = 256;           // k values per pass (4 per lane)
constexpr int GUARD_ROW = GUARD_CHUNK + 4; // LDS floats per candidate row (padded)

// Reference-order dot products for up to GUARD_GROUP candidate experts of one
// token (src/ds3_reference.c:424-434: acc += x[i]*w[i], i ascending, product
// and sum rounded separately).  Per 256-wide chunk the wave forms the exact
// products of every candidate (lane l: k = 4l..4l+3) into LDS with all loads
// of the chunk in flight together; lane c then adds candidate c's 256
// products in index order.  Returns the logit in lane c < nc.
__device__ float guard_recompute(const float *x, int K, int rtype, const uint8_t *rw, uint64_t rstride,
                                 const int *cand, int nc, float *prod, int lane)
{
#pragma clang fp contract(off)
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += GUARD_CHUNK) {
        const int kb = k0 + 4 * lane;
        float xv[4], wv[GUARD_GROUP][4];        // zero past K: adding +0 products changes no sum
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = kb + i < K ? x[kb + i] : 0.0f;
#pragma unroll
        for (int c = 0; c < GUARD_GROUP; c++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                wv[c][i] = (c < nc && kb + i < K) ? router_weight(rtype, rw, rstride, cand[c], kb + i) : 0.0f;
#pragma unroll
        for (int c = 0; c < GUARD_GROUP; c++) {
            if (c < nc) {
                float4 pr;
                pr.x = xv[0] * wv[c][0];
                pr.y = xv[1] * wv[c][1];
                pr.z = xv[2] * wv[c][2];
                pr.w = xv[3] * wv[c][3];
                *(float4 *)(prod + c * GUARD_ROW + 4 * lane) = pr;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (lane < nc) {
            const float *pr = prod + lane * GUARD_ROW;
            const int n = min(GUARD_CHUNK, (K - k0 + 3) & ~3);
            for (int i = 0; i < n; i += 4) {
                const float4 v = *(const float4 *)(pr + i);
                acc = acc + v.x;
                acc = acc + v.y;
                acc = acc + v.z;
                acc = acc + v.w;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    return acc;
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
                uint64_t rstride, int kc, float *__restrict__ part, float *__restrict__ wn)
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
            if (g == 0) wn[(int64_t)ks * E + 16 * nb + r] = v;
        }
    }
}

__global__ void __launch_bounds__(256) k_route(RouteArgs a)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (t >= a.T) return;                      // whole wave leaves together
    const int E = a.E;
    const int wv = threadIdx.x / WAVE;
    __shared__ float prod_s[4][GUARD_GROUP * GUARD_ROW];
    __shared__ int cand_s[4][ROUTE_MAX_E];
    __shared__ float exact_s[4][ROUTE_MAX_E];

    // logits: one row, or the sum of a.nparts split-K partial rows in order
    float l[ROUTE_EPL];
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) {
        const int e = lane + WAVE * j;
        float v = -INFINITY;
        if (e < E) {
            const float *lg = a.logits + (int64_t)t * a.logit_stride + e;
            v = lg[0];
        #pragma unroll 8
            for (int p = 1; p < a.nparts; p++) v += lg[(int64_t)p * a.part_stride];
        }
        l[j] = v;
    }

    int32_t *oi = a.idx + (int64_t)t * a.out_stride;
    float *os = a.scores + (int64_t)t * a.out_stride;
    bool ordered = false;          // selection already known from the logit order
    int sel_i = 0;

    if (a.x != nullptr) {
        // The need = min(k+1, E) largest logits in order (value desc, index
        // asc); lane r keeps round r's expert.
        const int need = min(a.k + 1, E);
        uint32_t taken = 0u;
        float prev = 0.f, kth = 0.f, min_gap = INFINITY;
        for (int r = 0; r < need; r++) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++) {
                const int e = lane + WAVE * j;
                if (!((taken >> j) & 1u) && e < E && (l[j] > bv || (l[j] == bv && e < bi))) { bv = l[j]; bi = e; }
            }
            wave_argmax(bv, bi);
            if (bi < E && (bi & (WAVE - 1)) == lane) taken |= 1u << (bi / WAVE);
            if (r > 0) min_gap = fminf(min_gap, prev - bv);
            prev = bv;
            if (r == a.k - 1) kth = bv;
            if (lane == r) sel_i = bi;
        }

        // Error bound from |x|_2 and the largest router row norm.
        const float *xt = a.x + (int64_t)t * a.K;
        float ss = 0.f;
#pragma unroll 8
        for (int i = lane; i < a.K; i += WAVE) ss += xt[i] * xt[i];
        ss = wave_sum(ss);
        float wmax = 0.f;
        for (int e = lane; e < E; e += WAVE) {
            float v = a.wnorm2[e];
#pragma unroll 8
            for (int p = 1; p < a.nparts; p++) v += a.wnorm2[(int64_t)p * E + e];
            wmax = fmaxf(wmax, v);
        }
        wmax = wave_max(wmax);
        const float tau = GUARD_C * 0x1.0p-24f * sqrtf(ss) * sqrtf(wmax);

        if (min_gap > fmaxf(2.0f * tau, 0x1.0p-19f)) {
            // Every neighbouring gap exceeds both roundings, so the reference
            // ranks these logits the same way; and a gap above 2^-19 keeps
            // their probabilities at least 16 ulp apart, so expf cannot tie
            // or reorder them: the order is the reference's (prob desc) order.
            // (A NaN gap fails the test and takes the general path.)
            ordered = sel_i >= 0 && sel_i < E;
            ordered = __all(ordered || lane >= a.k);
        } else {
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
                    const int pos = ns + __popcll(m & ((1ull << lane) - 1ull));
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
            int nc = 0;                         // compact the near ones in place
#pragma unroll
            for (int q = 0; q < ROUTE_EPL; q++) {
                const uint64_t nm = __ballot(near[q]);
                if (near[q]) cand_s[wv][nc + __popcll(nm & ((1ull << lane) - 1ull))] = my_e[q];
                nc += __popcll(nm);
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            for (int c0 = 0; c0 < nc; c0 += GUARD_GROUP) {
                const int n = min(GUARD_GROUP, nc - c0);
                const float v = guard_recompute(xt, a.K, a.rtype, a.rw, a.rstride, &cand_s[wv][c0], n,
                                                prod_s[wv], lane);
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
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) {
        const int e = lane + WAVE * j;
        p[j] = e < E ? expf(l[j] - mx) : 0.f;
        s += p[j];
    }
    s = wave_sum(s);
    const float inv = 1.0f / s;
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) p[j] *= inv;

    float sel_v = 0.f, ssum = 0.f;
    if (ordered) {
        // gather the probabilities of the already-ordered selection
        for (int r = 0; r < a.k; r++) {
            const int e = __shfl(sel_i, r, WAVE);
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++)
                if (lane + WAVE * j == e) v = p[j];
            v = wave_sum(v);
            ssum += v;                                            // sequential, in k order
            if (lane == r) sel_v = v;
        }
    } else {
        // Top-k by (prob desc, index asc).
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
    int ks = 512 / tiles;                      // ~512 workgroups
    if (ks < 1) ks = 1;
    if (ks > K / 64) ks = K / 64;
    if (ks > 32) ks = 32;
    while (ks > 1 && (K / 16) % ks != 0) ks--;  // equal chunks, multiples of 16
    return ks;
}

hipError_t launch_router_logits(const float *x, int T, int K, int E, int rtype, const uint8_t *rw, uint64_t rstride,
                                int nparts, float *part, float *wn, hipStream_t s)
{
    if (!router_mfma_ok(rtype, K, E, x, rw, rstride) || T <= 0 || nparts < 1 || (K / 16) % nparts != 0)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((T + RL_TOK - 1) / RL_TOK), (unsigned)nparts);
    hipLaunchKernelGGL(k_router_logits, grid, dim3(256), 0, s, x, T, K, E, rtype, rw, rstride, K / nparts, part, wn);
    return hipGetLastError();
}

hipError_t launch_route(const RouteArgs &a, hipStream_t s)
{
    if (a.T <= 0 || a.E <= 0 || a.E > ROUTE_MAX_E || a.k <= 0 || a.k > ROUTE_MAX_K || a.k > a.E || a.nparts < 1)
        return hipErrorInvalidValue;
    const int waves = 4;
    hipLaunchKernelGGL(k_route, dim3((unsigned)((a.T + waves - 1) / waves)), dim3(waves * WAVE), 0, s, a);
    return hipGetLastError();
}

}  // namespace ds3k
