// dequant.hip -- GGUF blocks -> f32, one lane per 32-weight unit.
//
// Every dequantised value is an exact product (Q6_K, Q8_0, F16) or an exact
// product minus an exact product rounded once (Q4_K), so this reproduces the
// reference's CPU dequantiser (src/ds3_reference.c:87-184) bit for bit.
#include "common.h"
#include "launch.h"

namespace ds3k {

__global__ void __launch_bounds__(256) k_dequant_q4k(const uint8_t *src, float *dst, int64_t n_units)
{
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_units) return;
    const int64_t b = u >> 3;
    const int c = (int)(u & 7);
    const uint8_t *blk = src + b * 144;
    const uint4 hdr = *(const uint4 *)blk;
    const uint4 q = *(const uint4 *)(blk + 16 + 16 * c);
    const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
    float sc0, mn0, sc1, mn1;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1), sc0, mn0);
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1) + 1, sc1, mn1);
    const float dl = d * sc0, ml = dmin * mn0, dh = d * sc1, mh = dmin * mn1;
    float *yl = dst + b * 256 + 64 * (c >> 1) + 16 * (c & 1);
    float *yh = yl + 32;
    const uint32_t qw[4] = { q.x, q.y, q.z, q.w };
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float a0, a1, a2, a3, b0, b1, b2, b3;
        cvt4(qw[i] & 0x0f0f0f0fu, a0, a1, a2, a3);
        cvt4((qw[i] >> 4) & 0x0f0f0f0fu, b0, b1, b2, b3);
        *(float4 *)(yl + 4 * i) = make_float4(dl * a0 - ml, dl * a1 - ml, dl * a2 - ml, dl * a3 - ml);
        *(float4 *)(yh + 4 * i) = make_float4(dh * b0 - mh, dh * b1 - mh, dh * b2 - mh, dh * b3 - mh);
    }
}

__global__ void __launch_bounds__(256) k_dequant_q6k(const uint8_t *src, float *dst, int64_t n_units)
{
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_units) return;
    const int64_t b = u >> 3;
    const int h = (int)((u >> 2) & 1), j = (int)(u & 3);
    const uint8_t *blk = src + b * 210;
    const uint2 lo = ld_u64_a2(blk + 64 * h + 8 * j);
    const uint2 hi = ld_u64_a2(blk + 64 * h + 32 + 8 * j);
    const uint2 qh = ld_u64_a2(blk + 128 + 32 * h + 8 * j);
    const uint2 scw = ld_u64_a2(blk + 192 + 8 * h);
    const float d = h2f(ld_u16(blk + 208));
    const int s0 = j >> 1;
    float *yb = dst + b * 256 + 128 * h + 8 * j;
    const uint32_t low[2] = { lo.x, lo.y }, hig[2] = { hi.x, hi.y }, hb[2] = { qh.x, qh.y };
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const float ds = d * (float)(int8_t)byte_of(t < 2 ? scw.x : scw.y, (s0 + 2 * t) & 3);
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t ql = (t & 1) ? hig[w] : low[w];
            const uint32_t nib = (t < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
            const uint32_t code = nib | (((hb[w] >> (2 * t)) & 0x03030303u) << 4);
            float c0, c1, c2, c3;
            cvt4(code, c0, c1, c2, c3);
            *(float4 *)(yb + 32 * t + 4 * w) =
                make_float4(ds * (c0 - 32.f), ds * (c1 - 32.f), ds * (c2 - 32.f), ds * (c3 - 32.f));
        }
    }
}

__global__ void __launch_bounds__(256) k_dequant_q80(const uint8_t *src, float *dst, int64_t n_units)
{
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_units) return;
    const uint8_t *blk = src + u * 34;
    const float d = h2f(ld_u16(blk));
    float *y = dst + u * 32;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t q = ld_u32_a2(blk + 2 + 4 * i);
        *(float4 *)(y + 4 * i) = make_float4((float)(int8_t)byte_of(q, 0) * d, (float)(int8_t)byte_of(q, 1) * d,
                                             (float)(int8_t)byte_of(q, 2) * d, (float)(int8_t)byte_of(q, 3) * d);
    }
}

__global__ void __launch_bounds__(256) k_dequant_f16(const uint16_t *src, float *dst, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = h2f(src[i]);
}

__global__ void __launch_bounds__(256) k_copy_f32(const float *src, float *dst, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

hipError_t launch_dequant(int type, const void *src, float *dst, int64_t n, hipStream_t s)
{
    const int tpb = 256;
    switch (type) {
    case T_Q4_K: {
        const int64_t nu = n / 32;
        hipLaunchKernelGGL(k_dequant_q4k, dim3((unsigned)((nu + tpb - 1) / tpb)), dim3(tpb), 0, s,
                           (const uint8_t *)src, dst, nu);
        break;
    }
    case T_Q6_K: {
        const int64_t nu = n / 32;
        hipLaunchKernelGGL(k_dequant_q6k, dim3((unsigned)((nu + tpb - 1) / tpb)), dim3(tpb), 0, s,
                           (const uint8_t *)src, dst, nu);
        break;
    }
    case T_Q8_0: {
        const int64_t nu = n / 32;
        hipLaunchKernelGGL(k_dequant_q80, dim3((unsigned)((nu + tpb - 1) / tpb)), dim3(tpb), 0, s,
                           (const uint8_t *)src, dst, nu);
        break;
    }
    case T_F16:
        hipLaunchKernelGGL(k_dequant_f16, dim3((unsigned)((n + tpb - 1) / tpb)), dim3(tpb), 0, s,
                           (const uint16_t *)src, dst, n);
        break;
    case T_F32:
        hipLaunchKernelGGL(k_copy_f32, dim3((unsigned)((n + tpb - 1) / tpb)), dim3(tpb), 0, s,
                           (const float *)src, dst, n);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace ds3k
