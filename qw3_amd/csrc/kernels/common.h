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
// The aligned address is p minus its low bits as pointer arithmetic, not an
// integer mask, so a pointer into LDS stays an LDS pointer (ds_read, not a
// flat load, which would also count against vmcnt).
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t *p)
{
    const uint32_t s = (uint32_t)((uintptr_t)p & 3);
    const uint32_t *q = (const uint32_t *)(p - s);
    return __builtin_amdgcn_alignbyte(q[1], q[0], s);
}

// Read 8 bytes at a 2-byte-aligned address (3 dword loads + 2 funnel shifts).
__device__ __forceinline__ uint2 ld_u64_a2(const uint8_t *p)
{
    const uint32_t s = (uint32_t)((uintptr_t)p & 3);
    const uint32_t *q = (const uint32_t *)(p - s);
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

// ---------------------------------------------------------------------------
// fp16 MFMA fragments straight from codes.  A code c (0..1023) becomes the
// fp16 value 1024 + c by OR-ing 0x6400 into its 16-bit lane (exponent 10,
// c in the mantissa); the weight is then one fused multiply-add
//   w = scale * (1024 + c) + (-(scale * (1024 + zero)) - min)
// computed at fp32 precision and rounded once to fp16 (v_fma_mix{lo,hi}_f16).
// The scale products are exact; only the folded constant rounds in fp32,
// ~1e-5 of a weight, far below the fp16 rounding of the result.
// ---------------------------------------------------------------------------
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

// 0x64006400 in a VGPR: with the mask in an SGPR, (x & mask) | magic is then
// a single v_and_or_b32 (gfx9 VOP3 takes no literal and one SGPR).
__device__ __forceinline__ uint32_t vgpr_magic()
{
    uint32_t v;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(v));
    return v;
}

// Four weights from one dword: codes of bytes 0 and 2 are x02 & mask, of
// bytes 1 and 3 x13 & mask (mask keeps the low code bits of each 16-bit
// lane).  Writes w[b0..b3] in byte order.
__device__ __forceinline__ void fma4(uint32_t x02, uint32_t x13, uint32_t mask, uint32_t mg, float sc, float c,
                                     _Float16 *w)
{
    const half2_t a = __builtin_bit_cast(half2_t, (x02 & mask) | mg);
    const half2_t b = __builtin_bit_cast(half2_t, (x13 & mask) | mg);
    w[0] = (_Float16)__builtin_fmaf(sc, (float)a[0], c);
    w[1] = (_Float16)__builtin_fmaf(sc, (float)b[0], c);
    w[2] = (_Float16)__builtin_fmaf(sc, (float)a[1], c);
    w[3] = (_Float16)__builtin_fmaf(sc, (float)b[1], c);
}

// ---------------------------------------------------------------------------
// Raw bytes of the two units (g, g+4) of one row in one 256-wide K step, held
// in registers while they are decoded.  load(base, sh, g) reads the step's
// quantised block of the row from base + sh, where base is 16-byte aligned
// (the row's staging area in LDS) and sh < 16 the block's byte offset in it;
// alignment is worked out on sh, never on pointer bits.  decode(hv) yields
// unit g + 4*hv exactly as unit_decode does.
// ---------------------------------------------------------------------------
template <int TYPE> struct RawUnits;

// First K index of the 8 weights that lane group g (lanes 16g..16g+15)
// supplies for K-slot q (0..7) of the 256-wide K step s, in RawUnits'
// decode_frags order: unit g + 4*(q/4), segment q%4.  The activation side of
// an MFMA reads the same 8 positions, so both operands share the K order.
template <int TYPE>
__device__ __forceinline__ int slot_k0(int s, int g, int q)
{
    const int c = g + 4 * (q >> 2), part = q & 3;
    if constexpr (TYPE == T_Q4_K)
        return 256 * s + 64 * (c >> 1) + 16 * (c & 1) + 8 * (part & 1) + 32 * (part >> 1);
    else if constexpr (TYPE == T_Q6_K)
        return 256 * s + 128 * (c >> 2) + 32 * part + 8 * (c & 3);
    else
        return 256 * s + 32 * c + 8 * part;
}

// Reads from LDS by byte address through inline asm, with their own
// s_waitcnt lgkmcnt(0) in the same statement.  The grouped kernels stream
// weights into LDS with global_load_lds DMAs; the compiler treats any LDS
// access it sees as possibly aliasing those and would wait for every DMA in
// flight, so the hot loops keep their LDS traffic in asm and order it
// themselves (vmcnt waits for the DMAs, lgkmcnt here, s_barrier).

template <> struct RawUnits<T_Q4_K> {
    uint4 hdr, q0, q1;
    __device__ __forceinline__ void load(const uint8_t *base, int sh, int g)
    {
        const uint8_t *blk = base + sh;              // sh == 0: Q4_K blocks are staged 16-byte aligned
        hdr = *(const uint4 *)blk;
        q0 = *(const uint4 *)(blk + 16 + 16 * g);
        q1 = *(const uint4 *)(blk + 16 + 16 * (g + 4));
    }
    // any alignment, straight from global memory (dword loads + funnel shifts)
    __device__ __forceinline__ void load_global(const uint8_t *blk, int g)
    {
        const uint8_t *p[3] = { blk, blk + 16 + 16 * g, blk + 16 + 16 * (g + 4) };
        uint32_t w[3][4];
#pragma unroll
        for (int f = 0; f < 3; f++)
#pragma unroll
            for (int i = 0; i < 4; i++) w[f][i] = ld_u32_a2(p[f] + 4 * i);
        hdr = make_uint4(w[0][0], w[0][1], w[0][2], w[0][3]);
        q0 = make_uint4(w[1][0], w[1][1], w[1][2], w[1][3]);
        q1 = make_uint4(w[2][0], w[2][1], w[2][2], w[2][3]);
    }
    // base: LDS byte address of the row's 16-byte aligned block
    __device__ __forceinline__ void load_lds(uint32_t base, int g)
    {
        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
        u4v h, a, b;
        asm volatile("ds_read_b128 %0, %3\n\t"
                     "ds_read_b128 %1, %4\n\t"
                     "ds_read_b128 %2, %5\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(h), "=&v"(a), "=&v"(b)
                     : "v"(base), "v"(base + 16 + 16 * g), "v"(base + 16 + 16 * (g + 4)));
        hdr = make_uint4(h.x, h.y, h.z, h.w);
        q0 = make_uint4(a.x, a.y, a.z, a.w);
        q1 = make_uint4(b.x, b.y, b.z, b.w);
    }
    // fragments p = 0..3 of unit g + 4*hv: low nibbles of bytes 0-7, 8-15,
    // then high nibbles of bytes 0-7, 8-15 (unit_decode's segment order)
    __device__ __forceinline__ void decode_frags(int hv, int g, half8_t (&fr)[4]) const
    {
        const uint4 q = hv ? q1 : q0;
        // (scale, min) of sub-blocks j, j+1 of unit g + 4hv, j = 2*(g>>1) + 4hv,
        // as two bytes each: get_scale_min_k4 (src/ds3_reference.c:76-85) on
        // the pair at once.  hv 0: low 6 bits of bytes j, j+4; hv 1: low
        // nibbles / high nibbles of bytes j+4 with the top 2 bits of bytes
        // j-4 / j.
        const uint32_t sh = (uint32_t)(g >> 1) * 16u;
        const uint32_t a = hdr.y >> sh, b = hdr.z >> sh;
        uint32_t scp, mp;
        if (hv == 0) {
            scp = a & 0x3f3fu;
            mp = b & 0x3f3fu;
        } else {
            const uint32_t cw = hdr.w >> sh;
            scp = (cw & 0x0f0fu) | ((a >> 2) & 0x3030u);
            mp = ((cw >> 4) & 0x0f0fu) | ((b >> 2) & 0x3030u);
        }
        const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
        const float dl = d * (float)(scp & 0xffu);
        const float dh16 = (d * 0.0625f) * (float)((scp >> 8) & 0xffu);   // exact: a power-of-two scale
        const float cl = -(1024.0f * dl) - dmin * (float)(mp & 0xffu);
        const float ch16 = -(1024.0f * dh16) - dmin * (float)((mp >> 8) & 0xffu);
        const uint32_t qw[4] = { q.x, q.y, q.z, q.w };
        const uint32_t mg = vgpr_magic();
#pragma unroll
        for (int p = 0; p < 4; p++) {
            _Float16 w[8];
#pragma unroll
            for (int dd = 0; dd < 2; dd++) {
                const uint32_t x = qw[2 * (p & 1) + dd];
                // high nibbles stay in place: fp16 1024 + 16*code, so the
                // scale is dh/16 (exact) and the constant -(64*dh + mh)
                if (p < 2) fma4(x, x >> 8, 0x000f000fu, mg, dl, cl, w + 4 * dd);
                else fma4(x, x >> 8, 0x00f000f0u, mg, dh16, ch16, w + 4 * dd);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) fr[p][i] = w[i];
        }
    }
    __device__ __forceinline__ void decode(int hv, int g, float (&w)[32]) const
    {
        const int c = g + 4 * hv;
        const uint4 q = hv ? q1 : q0;
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
    }
};

// Q6_K: all four 8-byte fields of a unit share the block's offset mod 4, so
// each is kept as 3 aligned dwords plus one shift and funnel-shifted at decode.
template <> struct RawUnits<T_Q6_K> {
    uint32_t f[2][4][3];      // [hv][ql_lo, ql_hi, qh, scales][dwords]
    uint32_t dw, sh;
    __device__ __forceinline__ void load(const uint8_t *base, int sh16, int g)
    {
        sh = (uint32_t)(sh16 & 3);
        const uint8_t *b4 = base + (sh16 & ~3);     // dword-aligned start at or below the block
#pragma unroll
        for (int hv = 0; hv < 2; hv++) {
            const int off[4] = { 64 * hv + 8 * g, 64 * hv + 32 + 8 * g, 128 + 32 * hv + 8 * g, 192 + 8 * hv };
#pragma unroll
            for (int fi = 0; fi < 4; fi++) {
                const uint32_t *q = (const uint32_t *)(b4 + off[fi]);
                f[hv][fi][0] = q[0]; f[hv][fi][1] = q[1]; f[hv][fi][2] = q[2];
            }
        }
        dw = ld_u16(base + sh16 + 208);
    }
    // base: LDS byte address of the 16-byte aligned chunk run holding the
    // block at byte offset sh16
    __device__ __forceinline__ void load_lds(uint32_t base, int sh16, int g)
    {
        sh = (uint32_t)(sh16 & 3);
        const uint32_t b4 = base + (uint32_t)(sh16 & ~3), bg = b4 + 8 * g;
        typedef uint32_t u2v __attribute__((ext_vector_type(2)));
        u2v r[12];
        uint32_t d16;
        // fields (dword offsets, three consecutive dwords each): from bg
        // (= b4 + 8g) ql_lo 0 | 16, ql_hi 8 | 24, qh 32 | 40 for half 0 | 1;
        // from b4 the scales 48 | 50
        asm volatile("ds_read2_b32 %0, %13 offset1:1\n\t"
                     "ds_read2_b32 %1, %13 offset0:2 offset1:8\n\t"
                     "ds_read2_b32 %2, %13 offset0:9 offset1:10\n\t"
                     "ds_read2_b32 %3, %13 offset0:32 offset1:33\n\t"
                     "ds_read2_b32 %4, %13 offset0:34 offset1:16\n\t"
                     "ds_read2_b32 %5, %13 offset0:17 offset1:18\n\t"
                     "ds_read2_b32 %6, %13 offset0:24 offset1:25\n\t"
                     "ds_read2_b32 %7, %13 offset0:26 offset1:40\n\t"
                     "ds_read2_b32 %8, %13 offset0:41 offset1:42\n\t"
                     "ds_read2_b32 %9, %14 offset0:48 offset1:49\n\t"
                     "ds_read2_b32 %10, %14 offset0:50 offset1:51\n\t"
                     "ds_read2_b32 %11, %14 offset0:52 offset1:52\n\t"
                     "ds_read_u16 %12, %15\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]),
                       "=&v"(r[7]), "=&v"(r[8]), "=&v"(r[9]), "=&v"(r[10]), "=&v"(r[11]), "=&v"(d16)
                     : "v"(bg), "v"(b4), "v"(base + (uint32_t)sh16 + 208));
        f[0][0][0] = r[0].x; f[0][0][1] = r[0].y; f[0][0][2] = r[1].x;
        f[0][1][0] = r[1].y; f[0][1][1] = r[2].x; f[0][1][2] = r[2].y;
        f[0][2][0] = r[3].x; f[0][2][1] = r[3].y; f[0][2][2] = r[4].x;
        f[1][0][0] = r[4].y; f[1][0][1] = r[5].x; f[1][0][2] = r[5].y;
        f[1][1][0] = r[6].x; f[1][1][1] = r[6].y; f[1][1][2] = r[7].x;
        f[1][2][0] = r[7].y; f[1][2][1] = r[8].x; f[1][2][2] = r[8].y;
        f[0][3][0] = r[9].x; f[0][3][1] = r[9].y; f[0][3][2] = r[10].x;
        f[1][3][0] = r[10].x; f[1][3][1] = r[10].y; f[1][3][2] = r[11].x;
        dw = d16;
    }
    // fragment t of unit (half hv, j = g): outputs 32t + 8g + i
    __device__ __forceinline__ void decode_frags(int hv, int g, half8_t (&fr)[4]) const
    {
        uint32_t v[4][2];
#pragma unroll
        for (int fi = 0; fi < 4; fi++) {
            v[fi][0] = __builtin_amdgcn_alignbyte(f[hv][fi][1], f[hv][fi][0], sh);
            v[fi][1] = __builtin_amdgcn_alignbyte(f[hv][fi][2], f[hv][fi][1], sh);
        }
        const float d = h2f(dw);
        const int s0 = g >> 1;
        const uint32_t mg = vgpr_magic();
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float ds = d * (float)(int8_t)byte_of(t < 2 ? v[3][0] : v[3][1], (s0 + 2 * t) & 3);
            const float cs = -1056.0f * ds;         // -(1024 + 32) * ds
            _Float16 w[8];
#pragma unroll
            for (int ww = 0; ww < 2; ww++) {
                const uint32_t ql = (t & 1) ? v[1][ww] : v[0][ww];
                const uint32_t qh = v[2][ww];
                // code = nibble | (2 high bits << 4) per byte, as one bitfield insert: the
                // nibble (bits 0-3 of ql for t < 2, bits 4-7 for t >= 2) under the mask,
                // qh shifted so that field t (bits 2t, 2t+1) lands on bits 4-5; bits 6-7
                // of each byte keep whatever falls there, and fma4's 6-bit mask drops them.
                // Bytes 0/2 and 1/3 feed the two fp16 lanes.
                const uint32_t nib = (t < 2) ? ql : (ql >> 4);
                const uint32_t hs = t == 0 ? qh << 4 : t == 1 ? qh << 2 : t == 2 ? qh : qh >> 2;
                const uint32_t code = (nib & 0x0f0f0f0fu) | (hs & 0xf0f0f0f0u);
                fma4(code, code >> 8, 0x003f003fu, mg, ds, cs, w + 4 * ww);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) fr[t][i] = w[i];
        }
    }
    __device__ __forceinline__ void decode(int hv, int g, float (&w)[32]) const
    {
        uint32_t v[4][2];
#pragma unroll
        for (int fi = 0; fi < 4; fi++) {
            v[fi][0] = __builtin_amdgcn_alignbyte(f[hv][fi][1], f[hv][fi][0], sh);
            v[fi][1] = __builtin_amdgcn_alignbyte(f[hv][fi][2], f[hv][fi][1], sh);
        }
        const float d = h2f(dw);
        const int s0 = g >> 1;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float ds = d * (float)(int8_t)byte_of(t < 2 ? v[3][0] : v[3][1], (s0 + 2 * t) & 3);
#pragma unroll
            for (int ww = 0; ww < 2; ww++) {
                const uint32_t ql = (t & 1) ? v[1][ww] : v[0][ww];
                const uint32_t nib = (t < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                const uint32_t code = nib | (((v[2][ww] >> (2 * t)) & 0x03030303u) << 4);
                float c0, c1, c2, c3;
                cvt4(code, c0, c1, c2, c3);
                w[8 * t + 4 * ww + 0] = ds * (c0 - 32.f); w[8 * t + 4 * ww + 1] = ds * (c1 - 32.f);
                w[8 * t + 4 * ww + 2] = ds * (c2 - 32.f); w[8 * t + 4 * ww + 3] = ds * (c3 - 32.f);
            }
        }
    }
};

// Q8_0: a 34-byte block at offset 0 or 2 mod 4 lies inside 9 aligned dwords.
template <> struct RawUnits<T_Q8_0> {
    uint32_t q[2][9];
    uint32_t sh[2];
    __device__ __forceinline__ void load(const uint8_t *base, int sh16, int g)
    {
#pragma unroll
        for (int hv = 0; hv < 2; hv++) {
            const int o = sh16 + (g + 4 * hv) * 34;  // the unit's 34-byte block
            sh[hv] = (uint32_t)(o & 3);
            const uint32_t *p = (const uint32_t *)(base + (o & ~3));
#pragma unroll
            for (int i = 0; i < 9; i++) q[hv][i] = p[i];
        }
    }
    // base: LDS byte address of the 16-byte aligned chunk run holding the
    // step's first block at byte offset sh16
    __device__ __forceinline__ void load_lds(uint32_t base, int sh16, int g)
    {
        typedef uint32_t u2v __attribute__((ext_vector_type(2)));
        uint32_t a4[2];
#pragma unroll
        for (int hv = 0; hv < 2; hv++) {
            const int o = sh16 + (g + 4 * hv) * 34;  // the unit's 34-byte block
            sh[hv] = (uint32_t)(o & 3);
            a4[hv] = base + (uint32_t)(o & ~3);
        }
        u2v r[8];
        uint32_t t0, t1;
        asm volatile("ds_read2_b32 %0, %10 offset1:1\n\t"
                     "ds_read2_b32 %1, %10 offset0:2 offset1:3\n\t"
                     "ds_read2_b32 %2, %10 offset0:4 offset1:5\n\t"
                     "ds_read2_b32 %3, %10 offset0:6 offset1:7\n\t"
                     "ds_read_b32 %8, %10 offset:32\n\t"
                     "ds_read2_b32 %4, %11 offset1:1\n\t"
                     "ds_read2_b32 %5, %11 offset0:2 offset1:3\n\t"
                     "ds_read2_b32 %6, %11 offset0:4 offset1:5\n\t"
                     "ds_read2_b32 %7, %11 offset0:6 offset1:7\n\t"
                     "ds_read_b32 %9, %11 offset:32\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]),
                       "=&v"(r[7]), "=&v"(t0), "=&v"(t1)
                     : "v"(a4[0]), "v"(a4[1]));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            q[0][2 * i] = r[i].x; q[0][2 * i + 1] = r[i].y;
            q[1][2 * i] = r[4 + i].x; q[1][2 * i + 1] = r[4 + i].y;
        }
        q[0][8] = t0;
        q[1][8] = t1;
    }
    __device__ __forceinline__ void decode_frags(int hv, int g, half8_t (&fr)[4]) const
    {
        (void)g;
        const bool al = sh[hv] == 0;
        const float d = h2f(al ? (q[hv][0] & 0xffffu) : (q[hv][0] >> 16));
        const float c = -1152.0f * d;               // codes stored as int8 + 128
        const uint32_t mg = vgpr_magic();
#pragma unroll
        for (int p = 0; p < 4; p++) {
            _Float16 w[8];
#pragma unroll
            for (int dd = 0; dd < 2; dd++) {
                const int i = 2 * p + dd;
                const uint32_t x =
                    (al ? __builtin_amdgcn_alignbyte(q[hv][i + 1], q[hv][i], 2) : q[hv][i + 1]) ^ 0x80808080u;
                fma4(x, x >> 8, 0x00ff00ffu, mg, d, c, w + 4 * dd);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) fr[p][i] = w[i];
        }
    }
    __device__ __forceinline__ void decode(int hv, int g, float (&w)[32]) const
    {
        (void)g;
        const bool al = sh[hv] == 0;      // block starts on a dword: d low half, codes at byte 2
        const float d = h2f(al ? (q[hv][0] & 0xffffu) : (q[hv][0] >> 16));
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t c = al ? __builtin_amdgcn_alignbyte(q[hv][i + 1], q[hv][i], 2) : q[hv][i + 1];
#pragma unroll
            for (int j = 0; j < 4; j++) w[4 * i + j] = (float)(int8_t)byte_of(c, j) * d;
        }
    }
};

// F32 rows: no register staging (64 floats per row would not fit); decode loads.
template <> struct RawUnits<T_F32> {
    const uint8_t *row;
    int s;
    __device__ __forceinline__ void load(const uint8_t *r, int ss, int g)
    {
        (void)g;
        row = r;
        s = ss;
    }
    __device__ __forceinline__ void decode(int hv, int g, float (&w)[32]) const
    {
        int k0[4];
        unit_decode<T_F32>(row, 8 * s + g + 4 * hv, w, k0);
    }
    __device__ __forceinline__ void decode_frags(int hv, int g, half8_t (&fr)[4]) const
    {
        float w[32];
        decode(hv, g, w);
#pragma unroll
        for (int p = 0; p < 4; p++)
#pragma unroll
            for (int i = 0; i < 8; i++) fr[p][i] = (_Float16)w[8 * p + i];
    }
};

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

// RMSNorm's reduction order, shared by k_rms_norm and the certified router's
// fused prologue so both produce the same bits: in a 256-thread workgroup,
// thread t sums the squares of its contiguous run of ceil(n / 256) elements in
// index order, wave_sum adds the 64 lane partials, and the four wave totals are
// added in wave order; the scale is 1 / sqrt(ss / n + eps).
constexpr int NORM_THREADS = 256;
__device__ __forceinline__ float norm_rms(const float (&part)[4], int n, float eps)
{
#pragma clang fp contract(off)
    const float ss = ((part[0] + part[1]) + part[2]) + part[3];
    return 1.0f / sqrtf(ss / (float)n + eps);
}

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
