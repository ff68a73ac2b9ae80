// rowstream.h -- streaming quantised rows through registers and LDS.
//
// Shared by the one-token GEMV (gemv.hip, k_gemv1) and the decode gate/up
// kernel (moe_decode.hip): consecutive rows of a Q4_K / Q6_K / Q8_0 matrix are
// one contiguous byte range, loaded with 16-byte asm loads by a 256-thread
// workgroup into register sets (G1Set) and written to LDS; each lane then
// dots unit lane + 64 q of a row with its x values, held in registers in
// unit_decode's order with their 8-element sums (g1_unit_dot), and a DPP
// wave sum gives the row's product (g1_wave_total).
#pragma once
#include "common.h"

namespace ds3k {

constexpr int G1_TPB = 256;
constexpr int G1_LOAD = G1_TPB * 16;            // bytes one load instruction of the workgroup covers

template <int TYPE> struct G1Row;               // row bytes per 2048 weights
template <> struct G1Row<T_Q4_K> { static constexpr int RB = 1152; };
template <> struct G1Row<T_Q6_K> { static constexpr int RB = 1680; };
template <> struct G1Row<T_Q8_0> { static constexpr int RB = 2176; };

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


// This lane's x values for units lane + 64 q (q < UPL) in unit_decode's order
// and their 8-element sums; afterwards every value is used once by an empty
// asm, so the compiler's wait for these loads (a vmcnt it counts without the
// asm loads it cannot see) sits here.  Callers issue their first row chunks
// before this, so that one wait covers both.
template <int TYPE, int UPL>
__device__ __forceinline__ void g1_load_x(const float *__restrict__ x, int lane, float (&xr)[UPL][32],
                                          float (&sx)[UPL][4])
{
#pragma unroll
    for (int q = 0; q < UPL; q++) {
        int k0[4];
        unit_k0<TYPE>(lane + 64 * q, k0);
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < 8; i++) xr[q][8 * s + i] = x[k0[s] + i];
    }
#pragma unroll
    for (int q = 0; q < UPL; q++)
#pragma unroll
        for (int s = 0; s < 4; s++) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) t += xr[q][8 * s + i];
            sx[q][s] = t;
        }
#pragma unroll
    for (int q = 0; q < UPL; q++)
#pragma unroll
        for (int s = 0; s < 4; s++) asm volatile("" ::"v"(sx[q][s]));
}

}  // namespace ds3k
