// common.h -- device helpers shared by the gfx950 MoE-FFN kernels.
//
// GGUF block formats (reference src/ds3_reference.c:59-184):
//   Q4_K 144 B / 256 w : d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16
//   Q6_K 210 B / 256 w : ql[128] @0, qh[64] @128, scales[16] int8 @192, d f16 @208
//   Q8_0  34 B /  32 w : d f16 @0, qs[32] int8 @2
//
// A "unit" is 32 weights of one row that one lane decodes together:
//   Q4_K  unit (b, c), c = 0..7: qs bytes 16c..16c+15 of block b; low
//         nibbles are weights 256b + 64(c/2) + 16(c%2) + i, high nibbles the
//         same + 32 (i = 0..15).
//   Q6_K  unit (b, h, j), h = 0..1, j = 0..3: weights 256b + 128h + 32t + 8j + i
//         (t = 0..3, i = 0..7), codes from ql[64h+8j+i], ql[64h+32+8j+i],
//         qh[32h+8j+i].
//   Q8_0  unit = one block: weights 32u + i.
//   F32   unit = 32 consecutive floats.
// Every row of K values has K/32 units; unit u of a K_K type is block u/8,
// sub-unit u%8.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"

namespace ds3k {

constexpr int WAVE = 64;

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);   // exact
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// Read 4 bytes at a 2-byte-aligned address with dword-aligned loads only.
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t *p)
{
    const uintptr_t a = (uintptr_t)p;
    const uint32_t *q = (const uint32_t *)(a & ~(uintptr_t)3);
    return __builtin_amdgcn_alignbyte(q[1], q[0], (uint32_t)(a & 3));
}

// Read 8 bytes at a 2-byte-aligned address (3 dword loads + 2 funnel shifts).
__device__ __forceinline__ uint2 ld_u64_a2(const uint8_t *p)
{
    const uintptr_t a = (uintptr_t)p;
    const uint32_t *q = (const uint32_t *)(a & ~(uintptr_t)3);
    const uint32_t s = (uint32_t)(a & 3);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s));
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p)
{
    return *(const uint16_t *)p;
}

// (scale, min) j of a Q4_K block from its 12 scale bytes held as 3 dwords
// (reference src/ds3_reference.c:76-85).
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                              float &sc, float &mn)
{
    const uint32_t s[3] = { s0, s1, s2 };
    uint32_t a, b;
    if (j < 4) {
        a = byte_of(s[j >> 2], j & 3) & 63u;
        b = byte_of(s[(j + 4) >> 2], (j + 4) & 3) & 63u;
    } else {
        const uint32_t hi = byte_of(s[(j + 4) >> 2], (j + 4) & 3);
        a = (hi & 15u) | ((byte_of(s[(j - 4) >> 2], (j - 4) & 3) >> 6) << 4);
        b = (hi >> 4) | ((byte_of(s[j >> 2], j & 3) >> 6) << 4);
    }
    sc = (float)a;
    mn = (float)b;
}

// ---------------------------------------------------------------------------
// Unit dot products for the fp32 GEMV paths.  x points at the row's K floats
// (global or LDS).  Q4_K / Q6_K / Q8_0 use sum_i x_i * code_i with the
// per-group scale applied once, which is exact algebra on exactly
// representable weights; only the rounding order differs from a
// weight-by-weight dot.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void cvt4(uint32_t w, float &a, float &b, float &c, float &d)
{
    // (float)((w >> 8i) & 0xff) selects v_cvt_f32_ubyte{i}
    a = (float)(w & 0xffu);
    b = (float)((w >> 8) & 0xffu);
    c = (float)((w >> 16) & 0xffu);
    d = (float)(w >> 24);
}

template <typename XP>
__device__ __forceinline__ float dot4(uint32_t codes, XP x)
{
    float a, b, c, d;
    cvt4(codes, a, b, c, d);
    return x[0] * a + x[1] * b + x[2] * c + x[3] * d;
}

template <typename XP>
__device__ __forceinline__ float sum4(XP x) { return x[0] + x[1] + x[2] + x[3]; }

// Q4_K unit (b, c): returns sum over its 32 weights of w * x.
__device__ __forceinline__ float unit_dot_q4k(const uint8_t *row, int u, const float *x)
{
    const int b = u >> 3, c = u & 7;
    const uint8_t *blk = row + (size_t)b * 144;
    const uint4 hdr = *(const uint4 *)blk;
    const uint4 q = *(const uint4 *)(blk + 16 + 16 * c);
    const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
    float sc0, mn0, sc1, mn1;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1), sc0, mn0);
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1) + 1, sc1, mn1);
    const float *xl = x + 256 * b + 64 * (c >> 1) + 16 * (c & 1);
    const float *xh = xl + 32;
    const uint32_t qw[4] = { q.x, q.y, q.z, q.w };
    float dl = 0.f, dh = 0.f, sl = 0.f, sh = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        dl += dot4(qw[i] & 0x0f0f0f0fu, xl + 4 * i);
        dh += dot4((qw[i] >> 4) & 0x0f0f0f0fu, xh + 4 * i);
        sl += sum4(xl + 4 * i);
        sh += sum4(xh + 4 * i);
    }
    return (d * sc0) * dl - (dmin * mn0) * sl + (d * sc1) * dh - (dmin * mn1) * sh;
}

// Q6_K unit (b, h, j).
__device__ __forceinline__ float unit_dot_q6k(const uint8_t *row, int u, const float *x)
{
    const int b = u >> 3, h = (u >> 2) & 1, j = u & 3;
    const uint8_t *blk = row + (size_t)b * 210;
    const uint2 lo = ld_u64_a2(blk + 64 * h + 8 * j);
    const uint2 hi = ld_u64_a2(blk + 64 * h + 32 + 8 * j);
    const uint2 qh = ld_u64_a2(blk + 128 + 32 * h + 8 * j);
    const uint2 scw = ld_u64_a2(blk + 192 + 8 * h);       // scales[8h .. 8h+7]
    const float d = h2f(ld_u16(blk + 208));
    const int s0 = j >> 1;                                  // group (8j)/16 within the half
    const float *xb = x + 256 * b + 128 * h + 8 * j;
    const uint32_t low[2] = { lo.x, lo.y }, hig[2] = { hi.x, hi.y }, hb[2] = { qh.x, qh.y };
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t sc_byte = byte_of(t < 2 ? scw.x : scw.y, (s0 + 2 * t) & 3);
        const float sc = (float)(int8_t)sc_byte;
        const float *xt = xb + 32 * t;
        float dc = 0.f, sx = 0.f;
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t ql = (t & 1) ? hig[w] : low[w];
            const uint32_t nib = (t < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
            const uint32_t two = (hb[w] >> (2 * t)) & 0x03030303u;
            const uint32_t code = nib | (two << 4);          // 0..63 per byte
            dc += dot4(code, xt + 4 * w);
            sx += sum4(xt + 4 * w);
        }
        acc += sc * (dc - 32.f * sx);
    }
    return d * acc;
}

// Q8_0 unit = block u.
__device__ __forceinline__ float unit_dot_q80(const uint8_t *row, int u, const float *x)
{
    const uint8_t *blk = row + (size_t)u * 34;
    const float d = h2f(ld_u16(blk));
    const float *xb = x + 32 * u;
    float dc = 0.f, sx = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t q = ld_u32_a2(blk + 2 + 4 * i) ^ 0x80808080u;   // int8 + 128
        dc += dot4(q, xb + 4 * i);
        sx += sum4(xb + 4 * i);
    }
    return d * (dc - 128.f * sx);
}

__device__ __forceinline__ float unit_dot_f32(const uint8_t *row, int u, const float *x)
{
    const float *w = (const float *)row + 32 * u;
    const float *xb = x + 32 * u;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) acc += w[i] * xb[i];
    return acc;
}

template <int TYPE>
__device__ __forceinline__ float unit_dot(const uint8_t *row, int u, const float *x)
{
    if constexpr (TYPE == T_Q4_K) return unit_dot_q4k(row, u, x);
    else if constexpr (TYPE == T_Q6_K) return unit_dot_q6k(row, u, x);
    else if constexpr (TYPE == T_Q8_0) return unit_dot_q80(row, u, x);
    else return unit_dot_f32(row, u, x);
}

// Decode one unit into w[32]; weights w[8s..8s+7] pair with x[k0[s] .. k0[s]+7].
template <int TYPE>
__device__ __forceinline__ void unit_decode(const uint8_t *row, int u, float (&w)[32], int (&k0)[4])
{
    if constexpr (TYPE == T_Q4_K) {
        const int b = u >> 3, c = u & 7;
        const uint8_t *blk = row + (size_t)b * 144;
        const uint4 hdr = *(const uint4 *)blk;
        const uint4 q = *(const uint4 *)(blk + 16 + 16 * c);
        const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
        float sc0, mn0, sc1, mn1;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1), sc0, mn0);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * (c >> 1) + 1, sc1, mn1);
        const float dl = d * sc0, ml = dmin * mn0, dh = d * sc1, mh = dmin * mn1;
        const uint32_t qw[4] = { q.x, q.y, q.z, q.w };
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float a0, a1, a2, a3;
            cvt4(qw[i] & 0x0f0f0f0fu, a0, a1, a2, a3);
            w[4 * i + 0] = dl * a0 - ml; w[4 * i + 1] = dl * a1 - ml;
            w[4 * i + 2] = dl * a2 - ml; w[4 * i + 3] = dl * a3 - ml;
            cvt4((qw[i] >> 4) & 0x0f0f0f0fu, a0, a1, a2, a3);
            w[16 + 4 * i + 0] = dh * a0 - mh; w[16 + 4 * i + 1] = dh * a1 - mh;
            w[16 + 4 * i + 2] = dh * a2 - mh; w[16 + 4 * i + 3] = dh * a3 - mh;
        }
        const int kl = 256 * b + 64 * (c >> 1) + 16 * (c & 1);
        k0[0] = kl; k0[1] = kl + 8; k0[2] = kl + 32; k0[3] = kl + 40;
    } else if constexpr (TYPE == T_Q6_K) {
        const int b = u >> 3, h = (u >> 2) & 1, j = u & 3;
        const uint8_t *blk = row + (size_t)b * 210;
        const uint2 lo = ld_u64_a2(blk + 64 * h + 8 * j);
        const uint2 hi = ld_u64_a2(blk + 64 * h + 32 + 8 * j);
        const uint2 qh = ld_u64_a2(blk + 128 + 32 * h + 8 * j);
        const uint2 scw = ld_u64_a2(blk + 192 + 8 * h);
        const float d = h2f(ld_u16(blk + 208));
        const int s0 = j >> 1;
        const uint32_t low[2] = { lo.x, lo.y }, hig[2] = { hi.x, hi.y }, hb[2] = { qh.x, qh.y };
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float ds = d * (float)(int8_t)byte_of(t < 2 ? scw.x : scw.y, (s0 + 2 * t) & 3);
#pragma unroll
            for (int ww = 0; ww < 2; ww++) {
                const uint32_t ql = (t & 1) ? hig[ww] : low[ww];
                const uint32_t nib = (t < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                const uint32_t code = nib | (((hb[ww] >> (2 * t)) & 0x03030303u) << 4);
                float c0, c1, c2, c3;
                cvt4(code, c0, c1, c2, c3);
                w[8 * t + 4 * ww + 0] = ds * (c0 - 32.f); w[8 * t + 4 * ww + 1] = ds * (c1 - 32.f);
                w[8 * t + 4 * ww + 2] = ds * (c2 - 32.f); w[8 * t + 4 * ww + 3] = ds * (c3 - 32.f);
            }
            k0[t] = 256 * b + 128 * h + 32 * t + 8 * j;
        }
    } else if constexpr (TYPE == T_Q8_0) {
        const uint8_t *blk = row + (size_t)u * 34;
        const float d = h2f(ld_u16(blk));
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q = ld_u32_a2(blk + 2 + 4 * i);
#pragma unroll
            for (int j = 0; j < 4; j++) w[4 * i + j] = (float)(int8_t)byte_of(q, j) * d;
        }
#pragma unroll
        for (int s = 0; s < 4; s++) k0[s] = 32 * u + 8 * s;
    } else {
        const float *src = (const float *)row + 32 * u;
#pragma unroll
        for (int i = 0; i < 32; i++) w[i] = src[i];
#pragma unroll
        for (int s = 0; s < 4; s++) k0[s] = 32 * u + 8 * s;
    }
}

// Sum over groups of G consecutive lanes (G a power of two <= 64); every lane
// of the group ends with the group total.
template <int G>
__device__ __forceinline__ float group_sum(float v)
{
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<WAVE>(v); }

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// silu(g) * u with the reference's formula (src/ds3_reference.c:436-448).
__device__ __forceinline__ float swiglu(float g, float u)
{
    return (g / (1.0f + expf(-g))) * u;
}

}  // namespace ds3k
