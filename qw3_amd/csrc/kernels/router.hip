// router.hip -- softmax + top-k + renormalisation, one wavefront per token.
//
// Semantics follow the reference oracle (src/ds3_reference.c:344-359 softmax,
// :466-490 top-k, :632-639 renorm): probabilities exp(l - max) / sum, k rounds
// of selection by (prob desc, index asc), then weights divided by their sum.
//
// Margin guard.  Router logits come from a parallel fp32 reduction, whose
// rounding differs from the reference's sequential sum.  To keep the selected
// experts (and their order) identical to the reference except for genuine
// ties, each token checks the gaps between its 9 largest logits against an
// error bound tau = 64 * 2^-24 * |x|_2 * max_e |W_e|_2.  If a gap is below
// 2*tau, every logit within 2*tau of the 9th is recomputed in the reference's
// order (i ascending, separate multiply and add roundings), and selection
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

// Reference-order dot product (src/ds3_reference.c:424-434): acc += x[i]*w[i],
// i ascending, product and sum rounded separately.
__device__ __attribute__((noinline)) float sequential_logit(const float *x, int K, int rtype,
                                                            const uint8_t *rw, uint64_t rstride, int e)
{
#pragma clang fp contract(off)
    float acc = 0.0f;
    if (rtype == T_F32) {
        const float *row = (const float *)(rw + (size_t)e * rstride);
        for (int i = 0; i < K; i += 4) {
            const float4 xv = *(const float4 *)(x + i);
            const float w0 = row[i], w1 = row[i + 1], w2 = row[i + 2], w3 = row[i + 3];
            acc = acc + xv.x * w0;
            acc = acc + xv.y * w1;
            acc = acc + xv.z * w2;
            acc = acc + xv.w * w3;
        }
    } else {
        for (int i = 0; i < K; i++) {
            const float p = x[i] * router_weight(rtype, rw, rstride, e, i);
            acc = acc + p;
        }
    }
    return acc;
}

__global__ void __launch_bounds__(256) k_route(RouteArgs a)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (t >= a.T) return;                      // whole wave leaves together
    const int E = a.E;
    const float *lg = a.logits + (int64_t)t * a.logit_stride;

    float l[ROUTE_EPL];
#pragma unroll
    for (int j = 0; j < ROUTE_EPL; j++) {
        const int e = lane + WAVE * j;
        l[j] = e < E ? lg[e] : -INFINITY;
    }

    if (a.x != nullptr) {
        // The need = min(k+1, E) largest logits, in order; track the smallest
        // gap between neighbours and the last value.
        const int need = min(a.k + 1, E);
        uint32_t taken = 0u;
        float prev = 0.f, last = 0.f, min_gap = INFINITY;
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
            last = bv;
        }

        // Error bound from |x|_2 and the largest router row norm.
        const float *xt = a.x + (int64_t)t * a.K;
        float ss = 0.f;
        for (int i = lane; i < a.K; i += WAVE) ss += xt[i] * xt[i];
        ss = wave_sum(ss);
        float wmax = 0.f;
        for (int e = lane; e < E; e += WAVE) wmax = fmaxf(wmax, a.wnorm2[e]);
        wmax = wave_max(wmax);
        const float tau = GUARD_C * 0x1.0p-24f * sqrtf(ss) * sqrtf(wmax);

        if (min_gap < 2.0f * tau) {
            const float floor_v = last - 2.0f * tau;
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++) {
                const int e = lane + WAVE * j;
                if (e < E && l[j] >= floor_v)
                    l[j] = sequential_logit(xt, a.K, a.rtype, a.rw, a.rstride, e);
            }
            if (lane == 0 && a.guard_count) atomicAdd(a.guard_count, 1);
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

    // Top-k by (prob desc, index asc).
    int32_t *oi = a.idx + (int64_t)t * a.out_stride;
    float *os = a.scores + (int64_t)t * a.out_stride;
    float sel_v = 0.f;
    int sel_i = 0;
    float ssum = 0.f;
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
        if ((bi & (WAVE - 1)) == lane) {                          // remove from later rounds
#pragma unroll
            for (int j = 0; j < ROUTE_EPL; j++)
                if (j == bi / WAVE) p[j] = -2.0f;
        }
        ssum += bv;                                               // sequential, in k order
        if (lane == r) { sel_v = bv; sel_i = bi; }
    }
    if (lane < a.k) {
        float w = sel_v;
        if (a.norm && ssum > 0.0f) w *= 1.0f / ssum;
        oi[lane] = sel_i;
        os[lane] = w;
    }
}

hipError_t launch_route(const RouteArgs &a, hipStream_t s)
{
    if (a.T <= 0 || a.E <= 0 || a.E > ROUTE_MAX_E || a.k <= 0 || a.k > ROUTE_MAX_K || a.k > a.E)
        return hipErrorInvalidValue;
    const int waves = 4;
    hipLaunchKernelGGL(k_route, dim3((unsigned)((a.T + waves - 1) / waves)), dim3(waves * WAVE), 0, s, a);
    return hipGetLastError();
}

}  // namespace ds3k
