// gemv.hip -- fp32 products with quantised weights, C[m][n] = A[m] . W[n].
//
// The general-purpose kernel behind the reference's vec_matmul_* and
// matmul_quantized_batch entry points (src/ds3_metal.h:90-161) and the router
// logits.  Lanes split K in 32-weight units; a group of G lanes owns one row
// and decodes each unit once for a tile of up to 8 tokens staged in LDS.
#include "common.h"
#include "launch.h"

namespace ds3k {

constexpr int GEMV_MT = 8;            // tokens per tile
constexpr int GEMV_TPB = 256;

template <int TYPE, int G>
__global__ void __launch_bounds__(GEMV_TPB)
k_gemv(const float *__restrict__ A, int64_t lda, const uint8_t *__restrict__ W, uint64_t stride,
       float *__restrict__ C, int64_t ldc, int M, int N, int K, int mt_max, int rows_per_wg,
       float *__restrict__ wnorm2)
{
    extern __shared__ float xs[];     // [mt][K]
    const int m0 = blockIdx.y * mt_max;
    const int mt = min(mt_max, M - m0);
    for (int i = threadIdx.x; i < mt * K; i += GEMV_TPB) {
        const int m = i / K, k = i - m * K;
        xs[i] = A[(int64_t)(m0 + m) * lda + k];
    }
    __syncthreads();

    constexpr int GPW = WAVE / G;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int gl = lane % G, grp = lane / G;
    const int U = K / 32;
    const bool want_norm = (wnorm2 != nullptr) && blockIdx.y == 0;
    for (int r = wave * GPW + grp; r < rows_per_wg; r += (GEMV_TPB / WAVE) * GPW) {
        const int n = blockIdx.x * rows_per_wg + r;
        const bool valid = n < N;
        float acc[GEMV_MT];
#pragma unroll
        for (int m = 0; m < GEMV_MT; m++) acc[m] = 0.f;
        float w2 = 0.f;
        if (valid) {
            const uint8_t *row = W + (size_t)n * stride;
            for (int u = gl; u < U; u += G) {
                float w[32];
                int k0[4];
                unit_decode<TYPE>(row, u, w, k0);
                if (want_norm) {
#pragma unroll
                    for (int i = 0; i < 32; i++) w2 += w[i] * w[i];
                }
#pragma unroll
                for (int m = 0; m < GEMV_MT; m++) {
                    if (m < mt) {
                        const float *xm = xs + m * K;
                        float a = acc[m];
#pragma unroll
                        for (int s = 0; s < 4; s++)
#pragma unroll
                            for (int i = 0; i < 8; i++) a += w[8 * s + i] * xm[k0[s] + i];
                        acc[m] = a;
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < GEMV_MT; m++) acc[m] = group_sum<G>(acc[m]);
        if (want_norm) w2 = group_sum<G>(w2);
        if (valid && gl == 0) {
#pragma unroll
            for (int m = 0; m < GEMV_MT; m++)
                if (m < mt) C[(int64_t)(m0 + m) * ldc + n] = acc[m];
            if (want_norm) wnorm2[n] = w2;
        }
    }
}

bool gemv_type_ok(int type, int K)
{
    if (K <= 0) return false;
    switch (type) {
    case T_F32:  return K % 32 == 0;
    case T_Q8_0: return K % 32 == 0;
    case T_Q4_K:
    case T_Q6_K: return K % 256 == 0;
    default:     return false;
    }
}

template <int TYPE>
static hipError_t gemv_type(int G, dim3 grid, size_t lds, hipStream_t s, const float *A, int64_t lda,
                            const uint8_t *w, uint64_t stride, float *C, int64_t ldc, int M, int N, int K,
                            int mt, int rpw, float *wn)
{
#define DS3_GEMV_CASE(GV)                                                                       \
    case GV:                                                                                    \
        hipLaunchKernelGGL((k_gemv<TYPE, GV>), grid, dim3(GEMV_TPB), lds, s, A, lda, w, stride, C, \
                           ldc, M, N, K, mt, rpw, wn);                                          \
        break;
    switch (G) {
        DS3_GEMV_CASE(1) DS3_GEMV_CASE(2) DS3_GEMV_CASE(4) DS3_GEMV_CASE(8)
        DS3_GEMV_CASE(16) DS3_GEMV_CASE(32) DS3_GEMV_CASE(64)
    default: return hipErrorInvalidValue;
    }
#undef DS3_GEMV_CASE
    return hipGetLastError();
}

// Lanes per row: the largest power of two dividing the unit count (no idle
// lanes), capped at 64.
static int lanes_per_row(int units)
{
    int g = 1;
    while (g < 64 && units % (2 * g) == 0) g *= 2;
    return g;
}

hipError_t launch_gemv(int type, const float *A, int64_t lda, const uint8_t *w, uint64_t stride,
                       float *C, int64_t ldc, int M, int N, int K, float *wnorm2, hipStream_t s)
{
    if (!gemv_type_ok(type, K) || M <= 0 || N <= 0) return hipErrorInvalidValue;
    const int G = lanes_per_row(K / 32);
    const int gpw = WAVE / G;
    const int rows_step = (GEMV_TPB / WAVE) * gpw;            // rows one pass of the WG covers
    int mt = GEMV_MT;
    while (mt > 1 && (size_t)mt * K * sizeof(float) > 64 * 1024) mt /= 2;
    const int gy = (M + mt - 1) / mt;
    // Aim for ~512 workgroups: fewer rows per WG when there are few token tiles.
    const int steps_total = (N + rows_step - 1) / rows_step;
    int want_x = 512 / gy;
    if (want_x < 1) want_x = 1;
    int steps_per_wg = (steps_total + want_x - 1) / want_x;
    if (steps_per_wg < 1) steps_per_wg = 1;
    const int rpw = steps_per_wg * rows_step;
    const dim3 grid((unsigned)((N + rpw - 1) / rpw), (unsigned)gy);
    const size_t lds = (size_t)mt * K * sizeof(float);
    switch (type) {
    case T_F32:  return gemv_type<T_F32>(G, grid, lds, s, A, lda, w, stride, C, ldc, M, N, K, mt, rpw, wnorm2);
    case T_Q8_0: return gemv_type<T_Q8_0>(G, grid, lds, s, A, lda, w, stride, C, ldc, M, N, K, mt, rpw, wnorm2);
    case T_Q4_K: return gemv_type<T_Q4_K>(G, grid, lds, s, A, lda, w, stride, C, ldc, M, N, K, mt, rpw, wnorm2);
    case T_Q6_K: return gemv_type<T_Q6_K>(G, grid, lds, s, A, lda, w, stride, C, ldc, M, N, K, mt, rpw, wnorm2);
    default:     return hipErrorInvalidValue;
    }
}

}  // namespace ds3k
