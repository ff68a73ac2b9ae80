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

constexpr int G1_TPB = 256;
constexpr int G1_LOAD = G1_TPB * 16;            // bytes one load instruction of the workgroup covers

template <int TYPE> struct G1Row;               // row bytes per 2048 weights
template <> struct G1Row<T_Q4_K> { static constexpr int RB = 1152; };
template <> struct G1Row<T_Q6_K> { static constexpr int RB = 1680; };
template <> struct G1Row<T_Q8_0> { static constexpr int RB = 2176; };

#ifndef DS3_G1_ROWS
#define DS3_G1_ROWS 8               // rows per chunk at K = 2048 (half at 4096)
#endif
#ifndef DS3_G1_WPC
#define DS3_G1_WPC 4                // persistent workgroups per CU
#endif
#ifndef DS3_G1_SETS
#define DS3_G1_SETS 2               // register sets of chunks in flight per workgroup
#endif

template <int TYPE, int UPL>
struct G1 {
    static constexpr int RB = G1Row<TYPE>::RB * UPL;             // bytes per row
    static constexpr int R = DS3_G1_ROWS / UPL;                  // rows per chunk
    static constexpr int CB = R * RB;                            // chunk bytes
    static constexpr int NL = (CB + G1_LOAD - 1) / G1_LOAD;      // 16-byte loads per thread and chunk
    static constexpr int BUF = NL * G1_LOAD;                     // LDS bytes per buffer
    static_assert(R % 4 == 0 && RB % 16 == 0, "whole rows per wave, 16-byte rows");
};

typedef uint32_t g1_u32x4 __attribute__((ext_vector_type(4)));

template <int NL>
struct G1Set {
    g1_u32x4 v[NL];
    // the chunk of cb bytes at byte offset off0.  Pieces past the chunk (the
    // last round of loads overshoots it) re-read its first 16 bytes, a line
    // the same instruction fetches anyway, instead of the next chunk's lines,
    // which another workgroup loads; pieces past the tensor's last 16 bytes
    // (the last chunk's missing rows) re-read those.  Neither is used.
    __device__ __forceinline__ void issue(const uint8_t *base, int64_t off0, int cb, int64_t lim)
    {
#pragma unroll
        for (int l = 0; l < NL; l++) {
            const int rel = 16 * (int)threadIdx.x + G1_LOAD * l;
            int64_t o = off0 + (rel < cb ? rel : 0);
            if (o > lim) o = lim;
            asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v[l]) : "v"(base + o) : "memory");
        }
    }
    // wait until at most N loads issued after this set's are outstanding
    template <int N>
    __device__ __forceinline__ void wait()
    {
        static_assert(N <= 63, "vmcnt field holds 0..63");
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
#pragma unroll
        for (int l = 0; l < NL; l++) asm volatile("" : "+v"(v[l]));
    }
    __device__ __forceinline__ void to_lds(uint8_t *buf) const
    {
#pragma unroll
        for (int l = 0; l < NL; l++) *(g1_u32x4 *)(buf + 16 * threadIdx.x + G1_LOAD * l) = v[l];
    }
};

// K positions of unit u's weights in unit_decode's order: w[8s + i] pairs
// with x[k0[s] + i].
template <int TYPE>
__device__ __forceinline__ void unit_k0(int u, int (&k0)[4])
{
    if constexpr (TYPE == T_Q4_K) {
        const int b = u >> 3, c = u & 7, kl = 256 * b + 64 * (c >> 1) + 16 * (c & 1);
        k0[0] = kl; k0[1] = kl + 8; k0[2] = kl + 32; k0[3] = kl + 40;
    } else if constexpr (TYPE == T_Q6_K) {
        const int b = u >> 3, h = (u >> 2) & 1, j = u & 3;
#pragma unroll
        for (int t = 0; t < 4; t++) k0[t] = 256 * b + 128 * h + 32 * t + 8 * j;
    } else {
#pragma unroll
        for (int s = 0; s < 4; s++) k0[s] = 32 * u + 8 * s;
    }
}

// Sum over the wavefront with the total in lane 63 (DPP, no LDS round trip):
// two quad swaps and row rotations by 4 and 8 leave every lane of a 16-lane
// row with the row's sum; row_bcast:15 adds row 0 into row 1 and row 2 into
// row 3, row_bcast:31 rows 0-1 into row 3.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float g1_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float g1_wave_total(float v)
{
    v = v + g1_dpp<0xB1>(v);           // quad_perm [1,0,3,2]
    v = v + g1_dpp<0x4E>(v);           // quad_perm [2,3,0,1]
    v = v + g1_dpp<0x124>(v);          // row_ror:4
    v = v + g1_dpp<0x128>(v);          // row_ror:8
    v = v + g1_dpp<0x142, 0xa>(v);     // row_bcast:15
    v = v + g1_dpp<0x143, 0xc>(v);     // row_bcast:31
    return v;
}

// One unit's dot with this lane's x values in unit_decode's order (xv[8s +
// i] pairs with the unit's weight 8s + i), factored like the reference's
// block dots: codes against x, then each sub-block's scale and offset once.
// sx[s] = xv[8s] + ... + xv[8s + 7], the same for every row, so it is
// computed once per lane.
template <int TYPE>
__device__ __forceinline__ float g1_unit_dot(const uint8_t *row, int u, const float (&xv)[32], const float (&sx)[4])
{
    if constexpr (TYPE == T_Q4_K) {
        const int b = u >> 3, c = u & 7;
        const uint8_t *blk = row + b * 144;
        const uint4 hdr = *(const uint4 *)blk;
        const uint4 q = *(const uint4 *)(blk + 16 + 16 * c);
        const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
        float sc0, mn0, sc1, mn1;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1), sc0, mn0);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1) + 1, sc1, mn1);
        const uint32_t qw[4] = { q.x, q.y, q.z, q.w };
        float dl = 0.f, dh = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            dl += dot4(qw[i] & 0x0f0f0f0fu, xv + 4 * i);
            dh += dot4((qw[i] >> 4) & 0x0f0f0f0fu, xv + 16 + 4 * i);
        }
        return (d * sc0) * dl - (dmin * mn0) * (sx[0] + sx[1]) + (d * sc1) * dh - (dmin * mn1) * (sx[2] + sx[3]);
    } else if constexpr (TYPE == T_Q6_K) {
        const int b = u >> 3, h = (u >> 2) & 1, j = u & 3;
        const uint8_t *blk = row + b * 210;
        const uint2 lo = ld_u64_a2(blk + 64 * h + 8 * j);
        const uint2 hi = ld_u64_a2(blk + 64 * h + 32 + 8 * j);
        const uint2 qh = ld_u64_a2(blk + 128 + 32 * h + 8 * j);
        const uint2 scw = ld_u64_a2(blk + 192 + 8 * h);
        const float d = h2f(ld_u16(blk + 208));
        const int s0 = j >> 1;
        const uint32_t low[2] = { lo.x, lo.y }, hig[2] = { hi.x, hi.y }, hb[2] = { qh.x, qh.y };
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float sc = (float)(int8_t)byte_of(t < 2 ? scw.x : scw.y, (s0 + 2 * t) & 3);
            float dc = 0.f;
#pragma unroll
            for (int ww = 0; ww < 2; ww++) {
                const uint32_t ql = (t & 1) ? hig[ww] : low[ww];
                const uint32_t nib = (t < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                dc += dot4(nib | (((hb[ww] >> (2 * t)) & 0x03030303u) << 4), xv + 8 * t + 4 * ww);
            }
            acc += sc * (dc - 32.f * sx[t]);
        }
        return d * acc;
    } else {
        static_assert(TYPE == T_Q8_0, "Q4_K, Q6_K or Q8_0");
        const uint8_t *blk = row + u * 34;
        const float d = h2f(ld_u16(blk));
        float dc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) dc += dot4(ld_u32_a2(blk + 2 + 4 * i) ^ 0x80808080u, xv + 4 * i);   // int8 + 128
        return d * (dc - 128.f * ((sx[0] + sx[1]) + (sx[2] + sx[3])));
    }
}

template <int TYPE, int UPL>
__global__ void __launch_bounds__(G1_TPB)
k_gemv1(const float *__restrict__ x, const uint8_t *__restrict__ W, float *__restrict__ y, int N, int nch)
{
    using P = G1<TYPE, UPL>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * P::BUF];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    float xr[UPL][32];
#pragma unroll
    for (int q = 0; q < UPL; q++) {
        int k0[4];
        unit_k0<TYPE>(lane + 64 * q, k0);
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < 8; i++) xr[q][8 * s + i] = x[k0[s] + i];
    }
    float sx[UPL][4];
#pragma unroll
    for (int q = 0; q < UPL; q++)
#pragma unroll
        for (int s = 0; s < 4; s++) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) t += xr[q][8 * s + i];
            sx[q][s] = t;
        }
    // x has landed before the first chunk's loads go out: the compiler's own
    // wait for x (it does not see the asm loads) then waits for x alone
#pragma unroll
    for (int q = 0; q < UPL; q++)
#pragma unroll
        for (int s = 0; s < 4; s++) asm volatile("" ::"v"(sx[q][s]));
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
