// elementwise.hip -- small memory-bound kernels around the expert products.
//
// gather / scatter / silu_mul / add / copy / zero keep the reference's
// elementwise entry points (metal/elementwise.metal:7-88, metal/moe.metal:95-127);
// combine is the deterministic per-token reduction of the prefill path: each
// output element sums its k routed contributions in top-k order
// (reference src/ds3_reference.c:674-678), so no float atomics are needed.
#include "common.h"
#include "launch.h"

namespace ds3k {

constexpr int EW_TPB = 256;

static dim3 grid1d(int64_t n) { return dim3((unsigned)((n + EW_TPB - 1) / EW_TPB)); }

__global__ void k_fill_zero(float *p, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// 16-byte stores (p 16-byte aligned), grid-stride over float4 units; the
// last n % 4 floats by thread 0 of workgroup 0.
__global__ void k_fill_zero4(float *p, int64_t n)
{
    const int64_t n4 = n / 4, stride = (int64_t)gridDim.x * EW_TPB;
    for (int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x; i < n4; i += stride)
        ((float4 *)p)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (blockIdx.x == 0 && threadIdx.x == 0)
        for (int64_t j = 4 * n4; j < n; j++) p[j] = 0.0f;
}

// Keeps one wave busy for `ticks` of the 100 MHz real-time counter, then
// exits; touches no memory.  Launched ahead of work whose kernels are timed
// with events, so that the host can enqueue that work before the stream
// reaches it.
__global__ void __launch_bounds__(64) k_hold(uint64_t ticks)
{
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(64);
}

__global__ void k_copy(const float *a, float *b, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i < n) b[i] = a[i];
}

__global__ void k_add(const float *a, const float *b, float *c, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i < n) c[i] = a[i] + b[i];
}

// Row ids outside [0, n_rows) (n_rows from the buffer size) are skipped.
__global__ void k_gather_rows(const float *src, const int32_t *ids, float *dst, int n_cols, int count, int64_t n_rows)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i >= (int64_t)n_cols * count) return;
    const int r = (int)(i / n_cols), c = (int)(i - (int64_t)r * n_cols);
    const int64_t row = ids[r];
    if (row >= 0 && row < n_rows) dst[i] = src[row * n_cols + c];
}

// dst[ids[i]][j] += scores[i] * src[i][j].  Rows of one call must be distinct
// (the reference's contract: one expert's token list), so there are no races.
__global__ void k_scatter_add(const float *src, const float *scores, const int32_t *ids, float *dst, int n_cols,
                              int count, int64_t n_rows)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i >= (int64_t)n_cols * count) return;
    const int r = (int)(i / n_cols), c = (int)(i - (int64_t)r * n_cols);
    const int64_t row = ids[r];
    if (row < 0 || row >= n_rows) return;
    float *d = dst + row * n_cols + c;
    *d = *d + scores[r] * src[i];
}

__global__ void k_silu_mul(const float *g, const float *u, float *out, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i < n) out[i] = swiglu(g[i], u[i]);
}

__global__ void k_axpy(const float *x, float w, float *y, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i < n) y[i] = y[i] + w * x[i];
}

__global__ void k_to_f16(const float *x, _Float16 *y, int64_t n4)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i >= n4) return;
    const float4 v = ((const float4 *)x)[i];
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    half4 h;
    h[0] = (_Float16)v.x; h[1] = (_Float16)v.y; h[2] = (_Float16)v.z; h[3] = (_Float16)v.w;
    ((half4 *)y)[i] = h;
}

// fp16 -> fp32, exact; one element per thread (any n, 2-byte aligned input).
__global__ void k_to_f32(const _Float16 *x, float *y, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * EW_TPB + threadIdx.x;
    if (i < n) y[i] = (float)x[i];
}

// out[t][j] = (acc ? out[t][j] : 0) + w_0 y[p_0][j] + ... in k order, then + residual.
// VEC consecutive columns per thread: 8 (16-byte y loads) or one.
template <int VEC>
__global__ void k_combine(const _Float16 *__restrict__ y, const int32_t *__restrict__ slot_pos,
                          const float *__restrict__ wts, int k, int N, float *__restrict__ out, int64_t ldo,
                          const float *__restrict__ residual, int accumulate)
{
#pragma clang fp contract(off)
    typedef float vec_t __attribute__((ext_vector_type(VEC)));
    typedef _Float16 hvec_t __attribute__((ext_vector_type(VEC)));
    const int t = blockIdx.y;
    const int j = (blockIdx.x * EW_TPB + threadIdx.x) * VEC;
    if (j >= N) return;
    constexpr int KMAX = VEC == 8 ? 8 : 16;   // slots whose loads are issued together
    static_assert(VEC == 8 || VEC == 1, "8 columns per thread or one");
    float *o = out + (int64_t)t * ldo + j;
    vec_t acc = accumulate ? *(const vec_t *)o : (vec_t)0.0f;
    for (int k0 = 0; k0 < k; k0 += KMAX) {
        vec_t v[KMAX];
        float w[KMAX];
        int p[KMAX];
#pragma unroll
        for (int kk = 0; kk < KMAX; kk++) {
            p[kk] = k0 + kk < k ? slot_pos[t * k + k0 + kk] : -1;
            w[kk] = p[kk] >= 0 ? wts[t * k + k0 + kk] : 0.0f;
            v[kk] = p[kk] >= 0 ? __builtin_convertvector(*(const hvec_t *)(y + (int64_t)p[kk] * N + j), vec_t)
                               : (vec_t)0.0f;
        }
#pragma unroll
        for (int kk = 0; kk < KMAX; kk++)
            if (p[kk] >= 0) acc = acc + w[kk] * v[kk];          // dropped slots add nothing
    }
    if (residual) acc = acc + *(const vec_t *)(residual + (int64_t)t * ldo + j);
    *(vec_t *)o = acc;
}

// RMSNorm of one row per workgroup (reference src/ds3_reference.c:329-342,
// metal/rms_norm.metal): out = x * (1 / sqrt(mean(x^2) + eps)) * weight, with
// the reference's formula (sum / n, + eps, 1 / sqrtf, then (x * rms) * w).
// The sum of squares is a fixed-order tree (norm_rms: per-thread contiguous
// runs, a wavefront butterfly, the four wave totals in order), not the
// reference's left-to-right chain, so rms can differ from it in the last bits,
// as the reference's Metal kernel's does; the result is the same on every call
// and the same as the certified router's fused prologue.
__global__ void __launch_bounds__(NORM_THREADS)
k_rms_norm(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ out, int n, float eps,
           int64_t ldx, int64_t ldo)
{
#pragma clang fp contract(off)
    __shared__ float part[NORM_THREADS / WAVE];
    const int64_t row = blockIdx.x;
    const float *xr = x + row * ldx;
    const int run = (n + NORM_THREADS - 1) / NORM_THREADS;
    const int b = threadIdx.x * run, e = min(b + run, n);
    float s = 0.f;
    for (int i = b; i < e; i++) {
        const float v = xr[i];
        s = s + v * v;
    }
    s = wave_sum(s);
    if ((threadIdx.x & (WAVE - 1)) == 0) part[threadIdx.x / WAVE] = s;
    __syncthreads();
    const float rms = norm_rms(part, n, eps);
    float *orow = out + row * ldo;
    for (int i = threadIdx.x; i < n; i += NORM_THREADS) orow[i] = xr[i] * rms * w[i];
}

hipError_t launch_rms_norm(const float *x, const float *w, float *out, int n, int n_rows, float eps, int64_t ldx,
                           int64_t ldo, hipStream_t s)
{
    if (n <= 0 || n_rows <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)n_rows), dim3(NORM_THREADS), 0, s, x, w, out, n, eps, ldx, ldo);
    return hipGetLastError();
}

hipError_t launch_fill_zero(float *p, int64_t n, hipStream_t s)
{
    if (((uintptr_t)p & 15) == 0) {
        // up to 1024 workgroups, each storing 4 KiB per pass
        const int64_t wg = (n / 4 + EW_TPB - 1) / EW_TPB;
        hipLaunchKernelGGL(k_fill_zero4, dim3((unsigned)(wg < 1 ? 1 : wg > 1024 ? 1024 : wg)), dim3(EW_TPB), 0, s, p,
                           n);
    }
    else hipLaunchKernelGGL(k_fill_zero, grid1d(n), dim3(EW_TPB), 0, s, p, n);
    return hipGetLastError();
}

hipError_t launch_hold(double us, hipStream_t s)
{
    if (!(us >= 0.0 && us <= 1e6)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_hold, dim3(1), dim3(64), 0, s, (uint64_t)(us * 100.0));
    return hipGetLastError();
}

hipError_t launch_copy(const float *a, float *b, int64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_copy, grid1d(n), dim3(EW_TPB), 0, s, a, b, n);
    return hipGetLastError();
}

hipError_t launch_add(const float *a, const float *b, float *c, int64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_add, grid1d(n), dim3(EW_TPB), 0, s, a, b, c, n);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const float *src, const int32_t *ids, float *dst, int n_cols, int count,
                              int64_t n_rows, hipStream_t s)
{
    hipLaunchKernelGGL(k_gather_rows, grid1d((int64_t)n_cols * count), dim3(EW_TPB), 0, s, src, ids, dst, n_cols,
                       count, n_rows);
    return hipGetLastError();
}

hipError_t launch_scatter_add(const float *src, const float *scores, const int32_t *ids, float *dst, int n_cols,
                              int count, int64_t n_rows, hipStream_t s)
{
    hipLaunchKernelGGL(k_scatter_add, grid1d((int64_t)n_cols * count), dim3(EW_TPB), 0, s, src, scores, ids, dst,
                       n_cols, count, n_rows);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *g, const float *u, float *out, int64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_silu_mul, grid1d(n), dim3(EW_TPB), 0, s, g, u, out, n);
    return hipGetLastError();
}

hipError_t launch_axpy(const float *x, float w, float *y, int64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_axpy, grid1d(n), dim3(EW_TPB), 0, s, x, w, y, n);
    return hipGetLastError();
}

hipError_t launch_to_f16(const float *x, _Float16 *y, int64_t n, hipStream_t s)
{
    if (n % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_to_f16, grid1d(n / 4), dim3(EW_TPB), 0, s, x, y, n / 4);
    return hipGetLastError();
}

hipError_t launch_to_f32(const _Float16 *x, float *y, int64_t n, hipStream_t s)
{
    if (n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_to_f32, grid1d(n), dim3(EW_TPB), 0, s, x, y, n);
    return hipGetLastError();
}

hipError_t launch_combine(const _Float16 *y, const int32_t *slot_pos, const float *wts, int T, int k, int N, float *out,
                          int64_t ldo, const float *residual, bool accumulate, hipStream_t s)
{
    // 8 columns per thread (16-byte y loads) whenever the rows allow it (the
    // grouped path's n_embd is a multiple of 128); one otherwise
    const bool vec8 = N % 8 == 0 && ldo % 4 == 0 &&
                      ((((uintptr_t)y) | ((uintptr_t)out) | ((uintptr_t)residual)) & 15) == 0;
    if (vec8) {
        const dim3 grid((unsigned)((N / 8 + EW_TPB - 1) / EW_TPB), (unsigned)T);
        hipLaunchKernelGGL(k_combine<8>, grid, dim3(EW_TPB), 0, s, y, slot_pos, wts, k, N, out, ldo, residual,
                           accumulate ? 1 : 0);
    } else {
        const dim3 grid((unsigned)((N + EW_TPB - 1) / EW_TPB), (unsigned)T);
        hipLaunchKernelGGL(k_combine<1>, grid, dim3(EW_TPB), 0, s, y, slot_pos, wts, k, N, out, ldo, residual,
                           accumulate ? 1 : 0);
    }
    return hipGetLastError();
}

}  // namespace ds3k
