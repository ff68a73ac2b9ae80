// gemv.hip -- fp32 products with quantised weights, C[m][n] = A[m] . W[n].
//
// The general-purpose kernel behind the reference's vec_matmul_* and
// matmul_quantized_batch entry points (src/ds3_metal.h:90-161) and the router
// logits.  Lanes split K in 32-weight units; a group of G lanes owns one row
// and decodes each unit once for a tile of up to 8 tokens staged in LDS.
//
// One token over long matrices (the output head, 151,936 x 2048, and the
// decode projections, src/ds3_engine.c:181-247) goes to k_gemv1 instead: the
// rows stream as one contiguous byte range per chunk of rows, not as the
// scattered unit loads of k_gemv.
#include "common.h"
#include "launch.h"
#include "rowstream.h"

namespace ds3k {

// ---------------------------------------------------------------------------
// k_gemv1: y[n] = x . W[n] for one token, Q4_K / Q6_K / Q8_0 rows of
// K = 2048 * UPL weights stored densely (row stride = row bytes) from a
// 16-byte aligned base.  Persistent workgroups walk chunks of R consecutive
// rows, one contiguous byte range each.  Every thread loads 16-byte pieces of
// a chunk into one of NS register sets in rotation (inline asm loads, waited
// by an asm s_waitcnt after which every register of the set is named), so
// NS - 1 chunks are in flight while one is decoded.  A landed chunk goes to
// one of two LDS buffers; each wave takes R/4 of its rows, each lane dots units
// lane + 64 q of a row from LDS with its x values, which stay in registers
// for the whole kernel with their 8-element sums (loaded once per
// workgroup), and a DPP wave sum gives the row's product.
// ---------------------------------------------------------------------------
bool gemv_type_ok(int type, int K);

#ifndef DS3_G1_ROWS
#define DS3_G1_ROWS 4               // rows per chunk at K = 2048 (half at 4096, at least 4)
#endif
#ifndef DS3_G1_WPC
#define DS3_G1_WPC 6                // persistent workgroups per CU
#endif
#ifndef DS3_G1_SETS
#define DS3_G1_SETS 2               // register sets of chunks in flight per workgroup
#endif

template <int TYPE, int UPL>
struct G1 {
    static constexpr int RB = G1Row<TYPE>::RB * UPL;             // bytes per row
    static constexpr int R = DS3_G1_ROWS / UPL < 4 ? 4 : DS3_G1_ROWS / UPL;   // rows per chunk (one per wave at least)
    static constexpr int CB = R * RB;                            // chunk bytes
    static constexpr int NL = (CB + G1_LOAD - 1) / G1_LOAD;      // 16-byte loads per thread and chunk
    static constexpr int BUF = NL * G1_LOAD;                     // LDS bytes per buffer
    static_assert(R % 4 == 0 && RB % 16 == 0, "whole rows per wave, 16-byte rows");
};

template <int TYPE, int UPL>
__global__ void __launch_bounds__(G1_TPB)
k_gemv1(const float *__restrict__ x, const uint8_t *__restrict__ W, float *__restrict__ y, int N, int nch)
{
    using P = G1<TYPE, UPL>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * P::BUF];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    float xr[UPL][32], sx[UPL][4];                    // loaded after the first chunks go out
    auto compute = [&](const uint8_t *buf, int c) {
        // one row at a time: four rows' decoded weights at once cost the second wave per SIMD
#pragma unroll 1
        for (int i = 0; i < P::R / 4; i++) {
            const int r = wave + 4 * i;
            float acc = 0.f;
#pragma unroll
            for (int q = 0; q < UPL; q++) acc += g1_unit_dot<TYPE>(buf + r * P::RB, lane + 64 * q, xr[q], sx[q]);
            acc = g1_wave_total(acc);
            const int n = c * P::R + r;
            if (lane == WAVE - 1 && n < N) y[n] = acc;
        }
    };
    const int G = (int)gridDim.x;
    int c = (int)blockIdx.x;
    const int64_t lim = (int64_t)N * P::RB - 16;
    // NS register sets in rotation: chunk k of this workgroup (c = blockIdx.x
    // + k G) loads into set k mod NS, NS - 1 chunks ahead of the one being
    // decoded, and goes to LDS buffer k mod 2
    constexpr int NS = DS3_G1_SETS;
    static_assert(NS >= 2 && (NS - 1) * P::NL <= 63, "register sets in flight vs the vmcnt field");
    G1Set<P::NL> S[NS];
#pragma unroll
    for (int j = 0; j < NS; j++) S[j].issue(W, (int64_t)min(c + j * G, nch - 1) * P::CB, P::CB, lim);
    // x after the first chunks: the wait for x (vmcnt 0, in issue order)
    // then covers them too, one memory latency instead of two
    g1_load_x<TYPE, UPL>(x, lane, xr, sx);
    bool more = true;
    for (int k = 0; more; k += NS) {
#pragma unroll
        for (int j = 0; j < NS; j++) {
            if (more) {                                   // uniform over the workgroup
                S[j].template wait<(NS - 1) * P::NL>();   // the other sets' loads went out after this one's
                uint8_t *buf = lds + ((k + j) & 1) * P::BUF;
                S[j].to_lds(buf);
                __syncthreads();                          // every wave is done with this buffer's previous chunk
                S[j].issue(W, (int64_t)min(c + NS * G, nch - 1) * P::CB, P::CB, lim);
                compute(buf, c);
                c += G;
                more = c < nch;
            }
        }
    }
    // every set still has loads in flight: wait for them, naming the registers
#pragma unroll
    for (int j = 0; j < NS; j++) S[j].template wait<0>();
}

template <int TYPE, int UPL>
static hipError_t gemv1_t(const float *x, const uint8_t *w, float *y, int N, hipStream_t s)
{
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    const int nch = (N + G1<TYPE, UPL>::R - 1) / G1<TYPE, UPL>::R;
    const int grid = nch < DS3_G1_WPC * n_cu ? nch : DS3_G1_WPC * n_cu;
    hipLaunchKernelGGL((k_gemv1<TYPE, UPL>), dim3((unsigned)grid), dim3(G1_TPB), 0, s, x, w, y, N, nch);
    return hipGetLastError();
}

// k_gemv1's shapes: one token, Q4_K / Q6_K / Q8_0, K = 2048 or 4096, dense
// rows from a 16-byte aligned base.
static bool gemv1_ok(int type, const uint8_t *w, uint64_t stride, int M, int K, const float *wnorm2)
{
    if (M != 1 || wnorm2 != nullptr || (K != 2048 && K != 4096) || ((uintptr_t)w & 15) != 0) return false;
    const int upl = K / 2048;
    switch (type) {
    case T_Q4_K: return stride == (uint64_t)G1Row<T_Q4_K>::RB * upl;
    case T_Q6_K: return stride == (uint64_t)G1Row<T_Q6_K>::RB * upl;
    case T_Q8_0: return stride == (uint64_t)G1Row<T_Q8_0>::RB * upl;
    default: return false;
    }
}

bool gemv1_path(int type, const uint8_t *w, uint64_t stride, int M, int K)
{
    return gemv_type_ok(type, K) && gemv1_ok(type, w, stride, M, K, nullptr);
}

static hipError_t launch_gemv1(int type, const float *x, const uint8_t *w, float *y, int N, int K, hipStream_t s)
{
    const bool two = K == 4096;
    switch (type) {
    case T_Q4_K: return two ? gemv1_t<T_Q4_K, 2>(x, w, y, N, s) : gemv1_t<T_Q4_K, 1>(x, w, y, N, s);
    case T_Q6_K: return two ? gemv1_t<T_Q6_K, 2>(x, w, y, N, s) : gemv1_t<T_Q6_K, 1>(x, w, y, N, s);
    case T_Q8_0: return two ? gemv1_t<T_Q8_0, 2>(x, w, y, N, s) : gemv1_t<T_Q8_0, 1>(x, w, y, N, s);
    default: return hipErrorInvalidValue;
    }
}

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
    if (gemv1_ok(type, w, stride, M, K, wnorm2)) return launch_gemv1(type, A, w, C, N, K, s);
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
