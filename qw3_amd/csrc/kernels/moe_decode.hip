// moe_decode.hip -- expert products for small token counts (decode).
//
// Bandwidth-bound GEMVs that stream each selected expert's quantised rows
// once, decoding in registers (reference decode kernels metal/moe.metal:140-391,
// host dispatch src/ds3_metal.m:2075-2290).  Two launches:
//   gate_up: h[slot][r] = silu(x_t . Wg_e[r]) * (x_t . Wu_e[r])
//   down:    out[t][j] = out[t][j] + w_0 y_0[j] + ... + w_{k-1} y_{k-1}[j]
//            with y_k[j] = h[slot_k] . Wd_{e_k}[j], summed in top-k order
//            (reference src/ds3_reference.c:674-678), no atomics.
#include "common.h"
#include "launch.h"

namespace ds3k {

__device__ __forceinline__ const uint8_t *expert_base(const uint8_t *base, const uint64_t *table, int e,
                                                      int which, uint64_t rows, uint64_t stride)
{
    return base + (table ? table[3 * e + which] : (uint64_t)e * rows * stride);
}

constexpr int DEC_TPB = 256;

// PAIR: h = swiglu(gate, up).  !PAIR: h = gate projection only, with expert
// offsets from table column `which` (unfused fallback for mixed types).
template <int GT, int G, bool PAIR>
__global__ void __launch_bounds__(DEC_TPB)
k_decode_gate_up(const float *__restrict__ x, int64_t ldx, const int32_t *__restrict__ idx, int n_used,
                 ExpertWeights ew, int K, int F, int rows_per_wg, int which, float *__restrict__ h)
{
    const int slot = blockIdx.y;
    const int t = slot / n_used;
    const int e = idx[slot];
    const uint8_t *wg = expert_base(ew.gate, ew.table, e, PAIR ? 0 : which, (uint64_t)F, ew.gate_stride);
    const uint8_t *wu = PAIR ? expert_base(ew.up, ew.table, e, 1, (uint64_t)F, ew.up_stride) : wg;
    const float *xt = x + (int64_t)t * ldx;

    constexpr int GPW = WAVE / G;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int gl = lane % G, grp = lane / G;
    const int U = K / 32;
    for (int rr = wave * GPW + grp; rr < rows_per_wg; rr += (DEC_TPB / WAVE) * GPW) {
        const int r = blockIdx.x * rows_per_wg + rr;
        const bool valid = r < F;
        float ag = 0.f, au = 0.f;
        if (valid) {
            const uint8_t *grow = wg + (size_t)r * ew.gate_stride;
            const uint8_t *urow = wu + (size_t)r * ew.up_stride;
            for (int u = gl; u < U; u += G) {
                ag += unit_dot<GT>(grow, u, xt);
                if (PAIR) au += unit_dot<GT>(urow, u, xt);
            }
        }
        ag = group_sum<G>(ag);
        if (PAIR) au = group_sum<G>(au);
        if (valid && gl == 0) h[(int64_t)slot * F + r] = PAIR ? swiglu(ag, au) : ag;
    }
}

template <int DT, int G>
__global__ void __launch_bounds__(1024)
k_decode_down(const float *__restrict__ h, const int32_t *__restrict__ idx, const float *__restrict__ wts,
              int n_used, ExpertWeights ew, int N, int F, int rows_per_wg, float *__restrict__ out,
              int64_t ldo, const float *__restrict__ residual, int accumulate)
{
    extern __shared__ float part[];            // [n_used][rows_per_wg]
    const int t = blockIdx.y;
    const int k = threadIdx.x / WAVE;          // one wave per selected expert
    const int slot = t * n_used + k;
    const int e = idx[slot];
    const uint8_t *wd = expert_base(ew.down, ew.table, e, 2, (uint64_t)N, ew.down_stride);
    const float *hs = h + (int64_t)slot * F;

    constexpr int GPW = WAVE / G;
    const int lane = threadIdx.x & (WAVE - 1);
    const int gl = lane % G, grp = lane / G;
    const int U = F / 32;
    for (int rr = grp; rr < rows_per_wg; rr += GPW) {
        const int j = blockIdx.x * rows_per_wg + rr;
        float acc = 0.f;
        if (j < N) {
            const uint8_t *row = wd + (size_t)j * ew.down_stride;
            for (int u = gl; u < U; u += G) acc += unit_dot<DT>(row, u, hs);
        }
        acc = group_sum<G>(acc);
        if (gl == 0) part[k * rows_per_wg + rr] = acc;
    }
    __syncthreads();
    for (int rr = threadIdx.x; rr < rows_per_wg; rr += blockDim.x) {
        const int j = blockIdx.x * rows_per_wg + rr;
        if (j >= N) continue;
        float *o = out + (int64_t)t * ldo + j;
        {
#pragma clang fp contract(off)
            float acc = accumulate ? *o : 0.0f;
            for (int kk = 0; kk < n_used; kk++) acc = acc + wts[t * n_used + kk] * part[kk * rows_per_wg + rr];
            if (residual) acc = acc + residual[(int64_t)t * ldo + j];
            *o = acc;
        }
    }
}

static int lanes_per_row(int units)
{
    int g = 1;
    while (g < 64 && units % (2 * g) == 0) g *= 2;
    return g;
}

#define DS3_G_SWITCH(G, CALL)                                                   \
    switch (G) {                                                                \
    case 1: { constexpr int GV = 1; CALL; } break;                              \
    case 2: { constexpr int GV = 2; CALL; } break;                              \
    case 4: { constexpr int GV = 4; CALL; } break;                              \
    case 8: { constexpr int GV = 8; CALL; } break;                              \
    case 16: { constexpr int GV = 16; CALL; } break;                            \
    case 32: { constexpr int GV = 32; CALL; } break;                            \
    case 64: { constexpr int GV = 64; CALL; } break;                            \
    default: return hipErrorInvalidValue;                                       \
    }

#define DS3_T_SWITCH(TY, CALL)                                                  \
    switch (TY) {                                                               \
    case T_F32: { constexpr int TV = T_F32; CALL; } break;                      \
    case T_Q8_0: { constexpr int TV = T_Q8_0; CALL; } break;                    \
    case T_Q4_K: { constexpr int TV = T_Q4_K; CALL; } break;                    \
    case T_Q6_K: { constexpr int TV = T_Q6_K; CALL; } break;                    \
    default: return hipErrorInvalidValue;                                       \
    }

static hipError_t decode_gate_up_impl(const float *x, int64_t ldx, const int32_t *idx, int n_slots, int n_used,
                                      const ExpertWeights &ew, int K, int F, float *h, bool pair, int which,
                                      hipStream_t s)
{
    if (!gemv_type_ok(ew.gate_type, K) || n_slots <= 0) return hipErrorInvalidValue;
    const int G = lanes_per_row(K / 32);
    const int rows_step = (DEC_TPB / WAVE) * (WAVE / G);
    // Two passes of the workgroup per block keeps ~768 WGs at T=1, F=768, G=64.
    int rpw = rows_step * 2;
    if (rpw > F) rpw = rows_step;
    const dim3 grid((unsigned)((F + rpw - 1) / rpw), (unsigned)n_slots);
    if (pair) {
        DS3_T_SWITCH(ew.gate_type, DS3_G_SWITCH(G, hipLaunchKernelGGL((k_decode_gate_up<TV, GV, true>), grid,
                                                                      dim3(DEC_TPB), 0, s, x, ldx, idx, n_used, ew,
                                                                      K, F, rpw, which, h)));
    } else {
        DS3_T_SWITCH(ew.gate_type, DS3_G_SWITCH(G, hipLaunchKernelGGL((k_decode_gate_up<TV, GV, false>), grid,
                                                                      dim3(DEC_TPB), 0, s, x, ldx, idx, n_used, ew,
                                                                      K, F, rpw, which, h)));
    }
    return hipGetLastError();
}

hipError_t launch_decode_gate_up(const float *x, int64_t ldx, const int32_t *idx, int n_slots, int n_used,
                                 const ExpertWeights &ew, int K, int F, float *h, hipStream_t s)
{
    if (ew.gate_type != ew.up_type) return hipErrorInvalidValue;
    return decode_gate_up_impl(x, ldx, idx, n_slots, n_used, ew, K, F, h, true, 0, s);
}

hipError_t launch_decode_proj(const float *x, int64_t ldx, const int32_t *idx, int n_slots, int n_used,
                              const ExpertWeights &ew, int which, int K, int F, float *out, hipStream_t s)
{
    return decode_gate_up_impl(x, ldx, idx, n_slots, n_used, ew, K, F, out, false, which, s);
}

hipError_t launch_decode_down(const float *h, const int32_t *idx, const float *wts, int T, int n_used,
                              const ExpertWeights &ew, int N, int F, float *out, int64_t ldo,
                              const float *residual, bool accumulate, hipStream_t s)
{
    if (!gemv_type_ok(ew.down_type, F) || T <= 0 || n_used <= 0 || n_used > 16) return hipErrorInvalidValue;
    const int G = lanes_per_row(F / 32);
    const int gpw = WAVE / G;
    const int rpw = gpw;                        // each wave covers its rows in one pass
    const dim3 grid((unsigned)((N + rpw - 1) / rpw), (unsigned)T);
    const size_t lds = (size_t)n_used * rpw * sizeof(float);
    DS3_T_SWITCH(ew.down_type, DS3_G_SWITCH(G, hipLaunchKernelGGL((k_decode_down<TV, GV>), grid, dim3(n_used * WAVE), lds, s,
                                                                  h, idx, wts, n_used, ew, N, F, rpw, out, ldo, residual,
                                                                  accumulate ? 1 : 0)));
    return hipGetLastError();
}

}  // namespace ds3k
