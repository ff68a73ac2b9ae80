// router.hip -- router logits in the reference's summation order, then
// softmax + top-k + renormalisation.
//
// Logits (src/ds3_reference.c:424-434): logit[t][e] = x[t][0]*W[e][0] +
// x[t][1]*W[e][1] + ..., summed with i ascending, each product and each
// partial sum rounded to fp32 on its own.  k_router_seq evaluates exactly that
// chain, one lane per (token, expert), so its logits are bit-identical to the
// reference's and top-k selection can differ from it only on exact ties.
// Router rows stored as F16 / Q8_0 / Q4_K / Q6_K are first expanded to FP32
// rows holding the values of the reference's FP32 copy (src/ds3_reference.c:
// 87-184).
//
// Selection (src/ds3_reference.c:344-359 softmax, :466-490 top-k, :632-639
// renorm): probabilities exp(l - max) / sum, k rounds of selection by (prob
// desc, index asc), then weights divided by their sum.  One wavefront per
// token.
#include <utility>

#include "route_select.h"

namespace ds3k {

// Element i of one router row as the reference's FP32 copy holds it
// (src/ds3_reference.c:87-184: the same products and roundings, no fusion).
template <int RT>
__device__ __forceinline__ float router_weight(const uint8_t *row, int i)
{
#pragma clang fp contract(off)
    if constexpr (RT == T_F32) {
        return ((const float *)row)[i];
    } else if constexpr (RT == T_F16) {
        return h2f(ld_u16(row + 2 * (size_t)i));
    } else if constexpr (RT == T_Q8_0) {
        const uint8_t *blk = row + (size_t)(i >> 5) * 34;
        return (float)(int8_t)blk[2 + (i & 31)] * h2f(ld_u16(blk));
    } else if constexpr (RT == T_Q4_K) {
        const uint8_t *blk = row + (size_t)(i >> 8) * 144;
        const int ib = i & 255, grp = ib >> 6, l = ib & 63;
        uint32_t sw[3];
#pragma unroll
        for (int w = 0; w < 3; w++)
            sw[w] = (uint32_t)blk[4 + 4 * w] | ((uint32_t)blk[5 + 4 * w] << 8) | ((uint32_t)blk[6 + 4 * w] << 16) |
                    ((uint32_t)blk[7 + 4 * w] << 24);
        float sc, mn;
        q4k_scale_min(sw[0], sw[1], sw[2], 2 * grp + (l >> 5), sc, mn);
        const int q = blk[16 + 32 * grp + (l & 31)];
        const float dl = h2f(ld_u16(blk)) * sc, ml = h2f(ld_u16(blk + 2)) * mn;
        return dl * (float)((l < 32) ? (q & 15) : (q >> 4)) - ml;
    } else {
        const uint8_t *blk = row + (size_t)(i >> 8) * 210;
        const int ib = i & 255, h = ib >> 7, t = (ib >> 5) & 3, l = ib & 31;
        const int qlb = blk[64 * h + l + 32 * (t & 1)];
        const int code = (((t < 2) ? (qlb & 15) : (qlb >> 4)) | (((blk[128 + 32 * h + l] >> (2 * t)) & 3) << 4)) - 32;
        const float sc = (float)(int8_t)blk[192 + 8 * h + (l >> 4) + 2 * t];
        return h2f(ld_u16(blk + 208)) * sc * (float)code;
    }
}

// FP32 copy of E router rows (stride K floats), element by element.
template <int RT>
__global__ void __launch_bounds__(256)
k_router_rows_f32(const uint8_t *__restrict__ rw, uint64_t rstride, int E, int K, float *__restrict__ out)
{
    const int e = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (e < E && i < K) out[(int64_t)e * K + i] = router_weight<RT>(rw + (size_t)e * rstride, i);
}

// ---------------------------------------------------------------------------
// Reference-order logits.  A workgroup covers 16 experts x 16 tokens: lane l
// of wave w sums token t0 + 4w + l/16 against expert e0 + l%16, one chain per
// lane.  The 16 W rows and 16 x rows stream through an LDS ring of D stages
// of 256-wide chunks by global_load_lds DMAs, so D-1 chunks are in flight
// while one is summed.  Rows are padded to 260 floats: the 16 lanes of each
// ds_read_b128 pass read 16 different W rows (16 different bank groups).  x
// is read one element per lane per 16-element block and reaches the other
// lanes of its 16-lane row by DPP broadcast (rs_sum).  With x16 != nullptr the workgroups also
// write the fp16 copy of x that the grouped products read (spread over the expert groups when
// the whole grid is resident at once).
// DW: DMA width in bytes, 16 (rows 16-byte aligned, K % 4 == 0) or 4.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define DS3_LDS __attribute__((address_space(3)))

constexpr int RS_CH = 256;                  // floats per row chunk
constexpr int RS_ROWB = (RS_CH + 4) * 4;    // bytes per padded LDS row
constexpr int RS_STAGE = 32 * RS_ROWB;      // 16 W rows + 16 x rows

// LDS reads of 16-element block blk (a constant once unrolled): 4 x 16
// bytes of the lane's W row (LDS byte address wa), and one element of its
// token's x row: lane l of each 16-lane row reads element l of the block
// (xa already includes 4 * (lane % 16)).  The 16 lanes of a row sum the
// same token, so the mul of element i takes x from lane i of the row by a
// DPP row broadcast instead of every lane reading all 16 elements: a
// quarter of the LDS bytes of 16-byte x reads per lane.
__device__ __forceinline__ void rs_read(int blk, uint32_t wa, uint32_t xa, u32x4 (&w)[4], uint32_t &x)
{
#pragma unroll
    for (int i = 0; i < 4; i++)
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(w[i]) : "v"(wa), "i"(64 * blk + 16 * i) : "memory");
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(x) : "v"(xa), "i"(64 * blk) : "memory");
}

// Wait until at most N LDS reads are outstanding: with the 5 reads of the
// next block issued after these, N = 5 releases exactly this block.
template <int N>
__device__ __forceinline__ void rs_wait(u32x4 (&w)[4], uint32_t &x)
{
    asm volatile("s_waitcnt lgkmcnt(%5)" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(x) : "i"(N));
}

// x[i] of the lane's token: element i of the block from lane i of the
// lane's 16-lane row (DPP row_newbcast, folded into the multiply).
template <int I>
__device__ __forceinline__ float rs_bcast(uint32_t x)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp((int)x, 0x150 + I, 0xf, 0xf, true));
}

// acc += x[i] * w[i] for the block's 16 elements in order, the product and
// the sum rounded separately (the folds run left to right).  One wave per
// SIMD sums its chains, so the time is the latency of the dependent adds:
// the 16 products are all issued first (the empty asm takes them as
// operands), and the adds then wait only on each other, not each on the
// multiply issued just before it.
template <int... I>
__device__ __forceinline__ void rs_sum_seq(float &acc, const u32x4 (&w)[4], uint32_t x,
                                           std::integer_sequence<int, I...>)
{
#pragma clang fp contract(off)
    float p[16];
    ((p[I] = rs_bcast<I>(x) * __uint_as_float(w[I / 4][I % 4])), ...);
    asm volatile("" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]), "+v"(p[4]), "+v"(p[5]), "+v"(p[6]),
                 "+v"(p[7]), "+v"(p[8]), "+v"(p[9]), "+v"(p[10]), "+v"(p[11]), "+v"(p[12]), "+v"(p[13]),
                 "+v"(p[14]), "+v"(p[15]));
    ((acc = acc + p[I]), ...);
}

__device__ __forceinline__ void rs_sum(float &acc, const u32x4 (&w)[4], uint32_t x)
{
    rs_sum_seq(acc, w, x, std::make_integer_sequence<int, 16>{});
}

// This wave's vector-memory loads (the ring's DMAs): wait until at most n
// remain.  Loads complete in issue order, so the oldest chunk is then done.
__device__ __forceinline__ void rs_vm_wait(int n)
{
    switch (n) {           // n is wave-uniform; above 40 (never used) waits for all
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
    case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
    case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
    case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
    case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
    case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    case 25: asm volatile("s_waitcnt vmcnt(25)" ::: "memory"); break;
    case 26: asm volatile("s_waitcnt vmcnt(26)" ::: "memory"); break;
    case 27: asm volatile("s_waitcnt vmcnt(27)" ::: "memory"); break;
    case 28: asm volatile("s_waitcnt vmcnt(28)" ::: "memory"); break;
    case 29: asm volatile("s_waitcnt vmcnt(29)" ::: "memory"); break;
    case 30: asm volatile("s_waitcnt vmcnt(30)" ::: "memory"); break;
    case 31: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
    case 32: asm volatile("s_waitcnt vmcnt(32)" ::: "memory"); break;
    case 33: asm volatile("s_waitcnt vmcnt(33)" ::: "memory"); break;
    case 34: asm volatile("s_waitcnt vmcnt(34)" ::: "memory"); break;
    case 35: asm volatile("s_waitcnt vmcnt(35)" ::: "memory"); break;
    case 36: asm volatile("s_waitcnt vmcnt(36)" ::: "memory"); break;
    case 37: asm volatile("s_waitcnt vmcnt(37)" ::: "memory"); break;
    case 38: asm volatile("s_waitcnt vmcnt(38)" ::: "memory"); break;
    case 39: asm volatile("s_waitcnt vmcnt(39)" ::: "memory"); break;
    case 40: asm volatile("s_waitcnt vmcnt(40)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

__device__ __forceinline__ void rs_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int DW, int D>
__global__ void __launch_bounds__(256)
k_router_seq(const float *__restrict__ x, int T, int K, int E, const float *__restrict__ w, int64_t wstride,
             float *__restrict__ logits, int64_t ldl, _Float16 *__restrict__ x16)
{
#pragma clang fp contract(off)
    constexpr int NDMA = 8 * (16 / DW);         // DMA instructions per wave per chunk (8 rows)
    static_assert(D >= 2 && (D - 2) * NDMA <= 32, "ring deeper than the vmcnt waits cover");
    __shared__ __attribute__((aligned(16))) uint8_t ring[D * RS_STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
    const int nch = (K + RS_CH - 1) / RS_CH;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(DS3_LDS void *)ring;

    // DMA sources of this wave's 8 rows: rows 8w..8w+7 of the stage, W rows
    // 0..15 then x rows 16..31 (rows past E / T repeat the last one)
    const float *src[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int r = 8 * wave + j;
        src[j] = r < 16 ? w + (int64_t)min(e0 + r, E - 1) * wstride : x + (int64_t)min(t0 + r - 16, T - 1) * K;
    }
    auto issue = [&](int c) {
        const uint32_t st = lds0 + (uint32_t)((c % D) * RS_STAGE);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t row = st + (uint32_t)((8 * wave + j) * RS_ROWB);
#pragma unroll
            for (int q = 0; q < 16 / DW; q++) {
                // lane element k of this instruction; past K it re-reads the row start (unused)
                const int k = c * RS_CH + (DW == 16 ? 4 * lane : 64 * q + lane);
                const float *p = src[j] + (k + DW / 4 - 1 < K ? k : 0);
                DS3_LDS void *dst = (DS3_LDS void *)(uintptr_t)(row + 256u * q);
                if constexpr (DW == 16) __builtin_amdgcn_global_load_lds(p, dst, 16, 0, 0);
                else __builtin_amdgcn_global_load_lds(p, dst, 4, 0, 0);
            }
        }
    };

    const int my_t = t0 + 4 * wave + (lane >> 4), my_e = e0 + (lane & 15);
    const uint32_t w_off = (uint32_t)((lane & 15) * RS_ROWB);
    const uint32_t x_off = (uint32_t)((16 + 4 * wave + (lane >> 4)) * RS_ROWB);
    const uint32_t xl_off = x_off + 4u * (uint32_t)(lane & 15);      // this lane's element of each x block
    // the fp16 copy of x: with one round of workgroups (D = 4, the whole grid
    // resident) chunk c by the expert group c mod gridDim.y, so the
    // conversion is spread over every workgroup of the token group; with
    // several rounds all of it by expert group 0 (measured faster there)
    const bool put16_any = x16 != nullptr;

#pragma unroll
    for (int c = 0; c < D - 1; c++)
        if (c < nch) issue(c);
    float acc = 0.0f;
    for (int c = 0; c < nch; c++) {
        rs_vm_wait(min(D - 2, nch - 1 - c) * NDMA);   // this wave's DMAs of chunk c have landed
        rs_barrier();                                 // everyone's have; stage (c-1) % D is free
        if (c + D - 1 < nch) issue(c + D - 1);
        const uint32_t st = lds0 + (uint32_t)((c % D) * RS_STAGE);
        const uint32_t wa = st + w_off, xa = st + x_off, xla = st + xl_off;
        const int kn = min(RS_CH, K - c * RS_CH);
        if (kn == RS_CH) {
            // 16-element blocks, two register sets: the reads of block i+1
            // are issued before block i is summed
            u32x4 w0[4], w1[4];
            uint32_t x0, x1;
            rs_read(0, wa, xla, w0, x0);
#pragma unroll
            for (int blk = 0; blk < RS_CH / 16; blk += 2) {
                rs_read(blk + 1, wa, xla, w1, x1);
                rs_wait<5>(w0, x0);
                rs_sum(acc, w0, x0);
                if (blk + 2 < RS_CH / 16) {
                    rs_read(blk + 2, wa, xla, w0, x0);
                    rs_wait<5>(w1, x1);
                } else {
                    rs_wait<0>(w1, x1);
                }
                rs_sum(acc, w1, x1);
            }
        } else {
            for (int k = 0; k < kn; k++) {
                uint32_t wv, xv;
                asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                             : "=&v"(wv), "=&v"(xv) : "v"(wa + 4u * k), "v"(xa + 4u * k) : "memory");
                acc = acc + __uint_as_float(xv) * __uint_as_float(wv);
            }
        }
        if (put16_any && (D >= 4 ? c % (int)gridDim.y == (int)blockIdx.y : blockIdx.y == 0)) {
            // thread: x row tid / 16 of the stage, 16 floats at 16 * (tid % 16)
            const int t = t0 + (tid >> 4), k0 = c * RS_CH + 16 * (tid & 15);
            if (t < T && k0 < K) {
                const uint32_t a = st + (uint32_t)((16 + (tid >> 4)) * RS_ROWB + 64 * (tid & 15));
                u32x4 v[4];
                asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:16\n\t"
                             "ds_read_b128 %2, %4 offset:32\n\tds_read_b128 %3, %4 offset:48\n\t"
                             "s_waitcnt lgkmcnt(0)"
                             : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]) : "v"(a) : "memory");
                _Float16 *d = x16 + (int64_t)t * K + k0;
                if (DW == 16 && k0 + 16 <= K) {
                    half8_t h0, h1;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        h0[i] = (_Float16)__uint_as_float(v[i / 4][i % 4]);
                        h1[i] = (_Float16)__uint_as_float(v[2 + i / 4][i % 4]);
                    }
                    *(half8_t *)d = h0;
                    *(half8_t *)(d + 8) = h1;
                } else {
#pragma unroll
                    for (int i = 0; i < 16; i++)
                        if (k0 + i < K) d[i] = (_Float16)__uint_as_float(v[i / 4][i % 4]);
                }
            }
        }
    }
    if (my_t < T && my_e < E) logits[(int64_t)my_t * ldl + my_e] = acc;
}

// ---------------------------------------------------------------------------
// Reference-order logits for few tokens.  Each logit is a chain of K
// dependent fp32 additions, which is the whole latency when few tokens are
// routed, so the multiplications leave the chain.  A workgroup of three waves
// covers EPW experts x 4 tokens: waves 1-2 form the exact products
// x[t][i]*W[e][i] of the next 128-wide chunk into an LDS product buffer while
// wave 0 (lane EPW*t + e) adds the current chunk's products in order.  W and x
// rows arrive by global_load_lds DMAs, issued by waves 1-2, through a ring of
// RSM_RD stages.  EPW = 4 spreads one token's 128 rows over 32 workgroups,
// EPW = 16 packs 4 tokens' work for more tokens.  Rows 16-byte aligned,
// K % 4 == 0.
// ---------------------------------------------------------------------------
constexpr int RSM_CH = 128;                         // floats per chunk
constexpr int RSM_RD = 8;                           // input ring stages (HBM latency at T = 1)
constexpr int RSM_ROW = RSM_CH * 4;                 // input row bytes (unpadded)
constexpr int RSM_PROWB = (RSM_CH + 4) * 4;         // product row bytes, padded
constexpr int RSM_MAX_T = 32;                       // larger batches use k_router_seq
template <int EPW> struct Rsm {
    static constexpr int IN_ROWS = EPW + 4;         // EPW W rows + 4 x rows
    static constexpr int NDMA = IN_ROWS / 4;        // DMAs per producer per chunk (2 rows each)
    static constexpr int IN = IN_ROWS * RSM_ROW;    // ring stage bytes
    static constexpr int P = 4 * EPW * RSM_PROWB;   // product buffer bytes
    static constexpr int LDS = RSM_RD * IN + 2 * P;
    static_assert(IN_ROWS % 4 == 0 && LDS <= 163840, "small router geometry");
};

__device__ __forceinline__ void lds_rd16(uint32_t a, u32x4 &v)
{
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a) : "memory");
}

__device__ __forceinline__ void lds_wr16(uint32_t a, const u32x4 &v)
{
    asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(v) : "memory");
}

__device__ __forceinline__ void lds_wait_all()
{
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Block blk (16 products = 64 bytes) of a product row at LDS address pa.
__device__ __forceinline__ void rsm_read(int blk, uint32_t pa, u32x4 (&v)[4])
{
#pragma unroll
    for (int i = 0; i < 4; i++)
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v[i]) : "v"(pa), "i"(64 * blk + 16 * i) : "memory");
}

template <int N>
__device__ __forceinline__ void rsm_wait(u32x4 (&v)[4])
{
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : "i"(N));
}

__device__ __forceinline__ void rsm_sum(float &acc, const u32x4 (&v)[4])
{
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc = acc + __uint_as_float(v[i][j]);
}

template <int EPW>
__global__ void __launch_bounds__(192)
k_router_small(const float *__restrict__ x, int T, int K, int E, const float *__restrict__ w, int64_t wstride,
               float *__restrict__ logits, int64_t ldl, RouteArgs topk, int *__restrict__ tickets)
{
#pragma clang fp contract(off)
    using G = Rsm<EPW>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[G::LDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * 4, e0 = blockIdx.y * EPW;
    const int nch = (K + RSM_CH - 1) / RSM_CH;
    const uint32_t in0 = (uint32_t)(uintptr_t)(DS3_LDS void *)lds;
    const uint32_t p0 = in0 + RSM_RD * G::IN;
    const int pw = wave - 1;                        // producer index (waves 1, 2)

    // producer pw moves input rows 2*NDMA*pw .. +2*NDMA-1, two per DMA
    // (lanes 0-31 the first, 32-63 the second): rows 0..EPW-1 W (experts),
    // then 4 x rows (tokens); rows past E / T repeat the last one (dropped)
    const float *src[G::NDMA];
#pragma unroll
    for (int i = 0; i < G::NDMA; i++) {
        const int r = 2 * (G::NDMA * pw + i) + (lane >> 5);
        src[i] = r < EPW ? w + (int64_t)min(e0 + r, E - 1) * wstride : x + (int64_t)min(t0 + r - EPW, T - 1) * K;
    }
    auto issue = [&](int c) {
        const uint32_t st = in0 + (uint32_t)((c % RSM_RD) * G::IN);
        const int k = c * RSM_CH + 4 * (lane & 31);
#pragma unroll
        for (int i = 0; i < G::NDMA; i++) {
            const float *p = src[i] + (k + 3 < K ? k : 0);      // past K: re-read the row start (unused)
            __builtin_amdgcn_global_load_lds(
                p, (DS3_LDS void *)(uintptr_t)(st + (uint32_t)(2 * (G::NDMA * pw + i) * RSM_ROW)), 16, 0, 0);
        }
    };
    // products of chunk c into buffer b: lane l of producer pw handles float4
    // k4 = l % 32 of experts 2pw + l/32 + 4s (s < EPW/4) for the 4 tokens;
    // all reads are issued before one wait
    auto produce = [&](int c, int b) {
        const uint32_t st = in0 + (uint32_t)((c % RSM_RD) * G::IN), pb = p0 + (uint32_t)(b * G::P);
        const int k4 = lane & 31, eb = 2 * pw + (lane >> 5);
        u32x4 wv[EPW / 4], xv[4];
#pragma unroll
        for (int sj = 0; sj < EPW / 4; sj++) lds_rd16(st + (uint32_t)((eb + 4 * sj) * RSM_ROW + 16 * k4), wv[sj]);
#pragma unroll
        for (int tk = 0; tk < 4; tk++) lds_rd16(st + (uint32_t)((EPW + tk) * RSM_ROW + 16 * k4), xv[tk]);
        lds_wait_all();
#pragma unroll
        for (int sj = 0; sj < EPW / 4; sj++)
#pragma unroll
            for (int tk = 0; tk < 4; tk++) {
                u32x4 pr;
#pragma unroll
                for (int q = 0; q < 4; q++) pr[q] = __float_as_uint(__uint_as_float(xv[tk][q]) * __uint_as_float(wv[sj][q]));
                lds_wr16(pb + (uint32_t)((EPW * tk + eb + 4 * sj) * RSM_PROWB + 16 * k4), pr);
            }
    };
    // wait until this producer's DMAs of chunk c have landed: NDMA per chunk,
    // chunks 0 .. issued-1 issued in order, so the NDMA * (issued - 1 - c)
    // newest may stay in flight
    int issued = 0;
    auto wait_chunk = [&](int c) { rs_vm_wait(G::NDMA * (issued - 1 - c)); };

    if (wave > 0) {
        for (; issued < RSM_RD && issued < nch; issued++) issue(issued);
        wait_chunk(0);
    }
    rs_barrier();
    if (wave > 0) {
        produce(0, 0);
        if (nch > 1) wait_chunk(1);
    }
    rs_barrier();
    float acc = 0.0f;
    const bool chain = lane < 4 * EPW;
    for (int c = 0; c < nch; c++) {
        if (wave == 0) {
            if (chain) {
                const uint32_t pa = p0 + (uint32_t)((c & 1) * G::P + lane * RSM_PROWB);
                const int kn = min(RSM_CH, K - c * RSM_CH);
                if (kn == RSM_CH) {
                    u32x4 v0[4], v1[4];
                    rsm_read(0, pa, v0);
#pragma unroll
                    for (int blk = 0; blk < RSM_CH / 16; blk += 2) {
                        rsm_read(blk + 1, pa, v1);
                        rsm_wait<4>(v0);
                        rsm_sum(acc, v0);
                        if (blk + 2 < RSM_CH / 16) {
                            rsm_read(blk + 2, pa, v0);
                            rsm_wait<4>(v1);
                        } else {
                            rsm_wait<0>(v1);
                        }
                        rsm_sum(acc, v1);
                    }
                } else {
                    for (int k = 0; k < kn; k++) {
                        uint32_t v;
                        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(pa + 4u * k) : "memory");
                        acc = acc + __uint_as_float(v);
                    }
                }
            }
        } else {
            if (c + 1 < nch) produce(c + 1, (c + 1) & 1);
            if (c + RSM_RD < nch) {
                issue(c + RSM_RD);                      // into the stage produce(c) read
                issued++;
            }
            if (c + 2 < nch) wait_chunk(c + 2);
        }
        rs_barrier();
    }
    const int t = t0 + lane / EPW, e = e0 + lane % EPW;
    if (wave == 0 && chain && t < T && e < E) logits[(int64_t)t * ldl + e] = acc;

    // Fused top-k: the last of the gridDim.y workgroups of this token group to
    // finish (a ticket per group, reset by that workgroup) routes its tokens
    // from the logits all of them wrote; fences make the stores visible
    // across XCDs before the ticket and to the reader after it.
    if (topk.idx != nullptr) {
        __shared__ int last_s;
        __threadfence();
        __syncthreads();
        if (tid == 0) last_s = atomicAdd(&tickets[blockIdx.x], 1) == (int)gridDim.y - 1;
        __syncthreads();
        if (last_s) {
            __threadfence();
            for (int tt = t0 + wave; tt < min(t0 + 4, T); tt += 3) route_token(topk, tt, lane);
            if (tid == 0) tickets[blockIdx.x] = 0;
        }
    }
}

__global__ void __launch_bounds__(256) k_route(RouteArgs a)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int t = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (t >= a.T) return;                      // whole wave leaves together
    route_token(a, t, lane);
}

// k_route for the grouped path, with the bucketing bitmaps: workgroup q
// routes tokens 4q .. 4q+3 (one per wave, as k_route) and writes its own row
// q of masks, one byte per expert: bit t % 4 of masks[t / 4][e] is set when
// token t chose expert e.  Rows are whole and private to their workgroup.
__global__ void __launch_bounds__(256) k_route_mark(RouteArgs a, uint8_t *__restrict__ masks)
{
    __shared__ uint32_t m_l[ROUTE_MAX_E];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) m_l[e] = 0u;
    __syncthreads();
    const int t = blockIdx.x * 4 + wave;
    if (t < a.T) {                                        // uniform over the wave
        const int e = route_token(a, t, lane);           // lane r < k: the expert it stored for rank r
        if (e >= 0 && e < a.E) atomicOr(&m_l[e], 1u << (t & 3));
    }
    __syncthreads();
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) masks[(int64_t)blockIdx.x * a.E + e] = (uint8_t)m_l[e];
}

hipError_t launch_route_mark(const RouteArgs &a, uint8_t *masks, hipStream_t s)
{
    if (a.T <= 0 || a.E <= 0 || a.E > ROUTE_MAX_E || a.k <= 0 || a.k > ROUTE_MAX_K || a.k > a.E)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_route_mark, dim3((unsigned)((a.T + 3) / 4)), dim3(256), 0, s, a, masks);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Certified router kernels (method and bound: route_select.h).
// ---------------------------------------------------------------------------

// S, B and fl32(S) for TG tokens x one expert.  Lane l of wave w covers
// elements (64 w + l) L .. + L - 1, K = 256 L.  With NORM the rows are first
// normalised in RMSNorm's reduction order (norm_rms: the same runs, butterfly
// and wave order), so every workgroup derives the same xn as k_rms_norm.
template <int L, int TG, bool NORM>
__global__ void __launch_bounds__(RC_THREADS)
k_router_sums(const float *__restrict__ x, int T, int K, int E, const float *__restrict__ w, int64_t wstride,
              float *__restrict__ logits, int64_t ldl, _Float16 *__restrict__ x16, CertArgs ca, NormPro np)
{
#pragma clang fp contract(off)
    static_assert(RC_THREADS == NORM_THREADS, "the fused norm needs RMSNorm's thread count");
    __shared__ float tot_s[TG][RC_WAVES];
    __shared__ float am_s[TG][RC_WAVES];
    __shared__ double sum_s[TG][RC_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * TG, e = blockIdx.y;
    const int k0 = tid * L;
    float wv[L], pv[TG][L];
    load_run<L>(w + (int64_t)e * wstride + k0, wv);
#pragma unroll
    for (int tt = 0; tt < TG; tt++) load_run<L>(x + (int64_t)min(t0 + tt, T - 1) * K + k0, pv[tt]);
    if constexpr (NORM) {
        float gv[L];
        load_run<L>(np.w + k0, gv);
#pragma unroll
        for (int tt = 0; tt < TG; tt++) {
            float q = 0.0f;
#pragma unroll
            for (int i = 0; i < L; i++) q = q + pv[tt][i] * pv[tt][i];
            q = wave_sum(q);
            if (lane == 0) am_s[tt][wave] = q;      // reused below, after a barrier
        }
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < TG; tt++) {
            const float rms = norm_rms(am_s[tt], K, np.eps);
#pragma unroll
            for (int i = 0; i < L; i++) pv[tt][i] = pv[tt][i] * rms * gv[i];
        }
        if (blockIdx.y == 0) {
#pragma unroll
            for (int tt = 0; tt < TG; tt++) {
                if (t0 + tt >= T) continue;
                float *d = np.xn + (int64_t)(t0 + tt) * K + k0;
#pragma unroll
                for (int i = 0; i < L; i++) d[i] = pv[tt][i];
            }
        }
        __syncthreads();                            // am_s is rewritten below
    }
    if (x16 != nullptr && blockIdx.y == 0) {
#pragma unroll
        for (int tt = 0; tt < TG; tt++) {
            if (t0 + tt >= T) continue;
            _Float16 *d = x16 + (int64_t)(t0 + tt) * K + k0;
#pragma unroll
            for (int i = 0; i < L; i++) d[i] = (_Float16)pv[tt][i];
        }
    }
    double sl[TG];
    float ex[TG];
#pragma unroll
    for (int tt = 0; tt < TG; tt++) {
        double s = 0.0;
        float r = 0.0f;
#pragma unroll
        for (int i = 0; i < L; i++) {
            const float p = pv[tt][i] * wv[i];      // the reference's rounded product
            s += (double)p;
            r = r + p;
            pv[tt][i] = r;                          // lane-local prefix
        }
        sl[tt] = s;
        // exclusive prefix of the lane totals, and the wave total
        ex[tt] = wave_incl_scan(dpp_f<0x138>(r));
        const float tot = readlane_f(ex[tt], 63) + readlane_f(r, 63);
        if (lane == 0) tot_s[tt][wave] = tot;
    }
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < TG; tt++) {
        float wbase = 0.0f;
        for (int v = 0; v < wave; v++) wbase = wbase + tot_s[tt][v];
        const float base = wbase + ex[tt];
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < L; i++) am = am + fabsf(base + pv[tt][i]);
        am = readlane_f(wave_incl_scan(am), 63);
        const double s = readlane_d(wave_incl_scan_f64(sl[tt]), 63);
        if (lane == 0) {
            am_s[tt][wave] = am;
            sum_s[tt][wave] = s;
        }
    }
    __syncthreads();
    if (tid < TG && t0 + tid < T) {
        const int t = t0 + tid;
        double s = sum_s[tid][0];
        float am = am_s[tid][0];
#pragma unroll
        for (int v = 1; v < RC_WAVES; v++) {
            s = s + sum_s[tid][v];
            am = am + am_s[tid][v];
        }
        ca.S[(int64_t)t * E + e] = s;
        ca.B[(int64_t)t * E + e] = am * ca.bfac + 1e-35f;
        logits[(int64_t)t * ldl + e] = (float)s;
    }
}

// Rank, certify, emit (and repair) the routing of TG tokens per workgroup:
// wave w takes token t0 + w on the one-wave path; a token it cannot certify
// goes through the whole workgroup's general path.
template <int TG>
__global__ void __launch_bounds__(RC_THREADS)
k_router_select(const float *__restrict__ x, int K, const float *__restrict__ w, int64_t wstride, CertArgs ca,
                RouteArgs a)
{
    extern __shared__ __attribute__((aligned(16))) float rc_prod[];
    __shared__ int fail_s[TG];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    const int t0 = blockIdx.x * TG;
    if (wave < TG) {
        const int t = t0 + wave;
        int e_rank;
        const bool ok = t < a.T && cert_select_wave(ca, a, t, true, lane, e_rank);
        if (lane == 0) fail_s[wave] = t < a.T && !ok ? 1 : 0;
    }
    __syncthreads();
    for (int tt = 0; tt < TG; tt++) {
        if (!fail_s[tt]) continue;                  // uniform over the workgroup
        cert_select_tokens<1>(x, K, w, wstride, ca, a, t0 + tt, true, rc_prod);
        __syncthreads();
    }
}


// bfac of the certified router for rows of K = 256 L values (see above):
// B = bfac * A_computed bounds |reference logit - S|.  0 when K is too long
// for the bound to stay tight.  The device's prefix of element i (lane-local
// prefix of <= L terms, a 6-level wave scan of lane totals, <= 3 wave totals)
// is within (3L + 14) u P + u |prefix| of the exact one, P = sum |p_i| <= 2 A;
// its sum of |prefix| runs through <= L + 10 roundings, and so does the
// fp64 S.
static double router_cert_bfac(int K)
{
    const double u = 0x1.0p-24;
    const double L = K / 256.0;
    const double d_a = 1.0 - 2.01 * K * (3.0 * L + 14.0) * u;
    if (d_a < 0.9 || K * u > 0.01) return 0.0;
    const double a_fac = (1.0 + u) / (1.0 - (L + 10.0) * u) / d_a;
    const double b = (u / (1.0 - K * u) + (L + 10.0) * 0x1.0p-52) * a_fac;
    return b * (1.0 + 0x1.0p-8);                                     // fp32 product bfac * A
}

bool router_cert_ok(int K, int E, int k)
{
    return K % 256 == 0 && K >= 256 && K <= 4096 && E >= 1 && E <= ROUTE_MAX_E && k >= 1 && k <= E &&
           k + 1 <= WAVE && router_cert_bfac(K) > 0.0;
}

size_t router_cert_scratch(int T, int E) { return (size_t)T * E * (sizeof(double) + sizeof(float)) + 256; }

template <int L, int TG>
static void cert_sums(const float *x, int T, int K, int E, const float *w, int64_t wstride, float *logits,
                      int64_t ldl, _Float16 *x16, const CertArgs &ca, const NormPro *np, hipStream_t s)
{
    const dim3 grid((unsigned)((T + TG - 1) / TG), (unsigned)E);
    if (np != nullptr)
        hipLaunchKernelGGL((k_router_sums<L, TG, true>), grid, dim3(RC_THREADS), 0, s, x, T, K, E, w, wstride, logits,
                           ldl, x16, ca, *np);
    else
        hipLaunchKernelGGL((k_router_sums<L, TG, false>), grid, dim3(RC_THREADS), 0, s, x, T, K, E, w, wstride,
                           logits, ldl, x16, ca, NormPro{});
}

template <int TG>
static void cert_select(const float *x, int T, int K, const float *w, int64_t wstride, const CertArgs &ca,
                        const RouteArgs &ra, hipStream_t s)
{
    const size_t lds = (size_t)ca.nb * (K + 4) * sizeof(float);
    hipLaunchKernelGGL((k_router_select<TG>), dim3((unsigned)((T + TG - 1) / TG)), dim3(RC_THREADS), lds, s, x, K, w,
                       wstride, ca, ra);
}

hipError_t router_cert_sel(int T, int K, int E, int k, int rtype, const uint8_t *rw, uint64_t rstride, float *wf32,
                           void *scratch, unsigned long long *stats, int nb, CertSel *out)
{
    if (T <= 0 || !router_cert_ok(K, E, k) || !router_seq_type_ok(rtype, K) || ((uintptr_t)scratch & 7) != 0)
        return hipErrorInvalidValue;
    const bool f32_direct = rtype == T_F32 && rstride % 16 == 0 && ((uintptr_t)rw & 15) == 0;
    if (!f32_direct && (wf32 == nullptr || ((uintptr_t)wf32 & 15) != 0)) return hipErrorInvalidValue;
    out->w = f32_direct ? (const float *)rw : wf32;
    out->wstride = f32_direct ? (int64_t)(rstride / 4) : (int64_t)K;
    CertArgs &ca = out->ca;
    ca.S = (double *)scratch;
    ca.B = (float *)((uint8_t *)scratch + (((size_t)T * E * sizeof(double) + 255) & ~(size_t)255));
    ca.bfac = (float)router_cert_bfac(K);
    ca.stats = stats;
    ca.nb = nb < 1 ? 1 : nb;
    return hipSuccess;
}

hipError_t launch_router_cert(const float *x, int T, int K, int E, int rtype, const uint8_t *rw, uint64_t rstride,
                              float *wf32, float *logits, int64_t ldl, _Float16 *x16, const RouteArgs &ra,
                              void *scratch, unsigned long long *stats, int phases, hipStream_t s,
                              const NormPro *norm)
{
    if (ra.logits != logits || ra.logit_stride != ldl || ra.T != T || ra.E != E || ra.idx == nullptr)
        return hipErrorInvalidValue;
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)x16 & 15) != 0) return hipErrorInvalidValue;
    if (norm != nullptr &&
        (phases != 1 || norm->w == nullptr || norm->xn == nullptr || ((uintptr_t)norm->w & 15) != 0 ||
         ((uintptr_t)norm->xn & 15) != 0 || !(norm->eps >= 0.0f)))
        return hipErrorInvalidValue;
    // repair batch: up to 13 candidate rows (about 104 KiB of LDS) while one
    // token group is routed, up to 4 (~32 KiB) when several workgroups share CUs
    const int rowb = (K + 4) * (int)sizeof(float);
    CertSel cs;
    hipError_t e = router_cert_sel(T, K, E, ra.k, rtype, rw, rstride, wf32, scratch, stats,
                                   T <= 4 ? min(13, 106496 / rowb) : min(4, 33792 / rowb), &cs);
    if (e != hipSuccess) return e;
    if ((const float *)rw != cs.w && (phases & 1)) {
        e = launch_router_rows(rtype, rw, rstride, E, K, wf32, s);
        if (e != hipSuccess) return e;
    }
    const float *w = cs.w;
    const int64_t wstride = cs.wstride;
    const CertArgs &ca = cs.ca;
    const int TG = T == 1 ? 1 : T == 2 ? 2 : 4;
#define DS3_CERT_SUMS(LV)                                                                        \
    do {                                                                                         \
        if (TG == 1) cert_sums<LV, 1>(x, T, K, E, w, wstride, logits, ldl, x16, ca, norm, s);          \
        else if (TG == 2) cert_sums<LV, 2>(x, T, K, E, w, wstride, logits, ldl, x16, ca, norm, s);     \
        else cert_sums<LV, 4>(x, T, K, E, w, wstride, logits, ldl, x16, ca, norm, s);                  \
    } while (0)
    if (phases & 1) switch (K / 256) {
    case 1: DS3_CERT_SUMS(1); break;
    case 2: DS3_CERT_SUMS(2); break;
    case 3: DS3_CERT_SUMS(3); break;
    case 4: DS3_CERT_SUMS(4); break;
    case 5: DS3_CERT_SUMS(5); break;
    case 6: DS3_CERT_SUMS(6); break;
    case 7: DS3_CERT_SUMS(7); break;
    case 8: DS3_CERT_SUMS(8); break;
    case 9: DS3_CERT_SUMS(9); break;
    case 10: DS3_CERT_SUMS(10); break;
    case 11: DS3_CERT_SUMS(11); break;
    case 12: DS3_CERT_SUMS(12); break;
    case 13: DS3_CERT_SUMS(13); break;
    case 14: DS3_CERT_SUMS(14); break;
    case 15: DS3_CERT_SUMS(15); break;
    case 16: DS3_CERT_SUMS(16); break;
    default: return hipErrorInvalidValue;
    }
#undef DS3_CERT_SUMS
    e = hipGetLastError();
    if (e != hipSuccess || !(phases & 2)) return e;
    if (TG == 1) cert_select<1>(x, T, K, w, wstride, ca, ra, s);
    else if (TG == 2) cert_select<2>(x, T, K, w, wstride, ca, ra, s);
    else cert_select<4>(x, T, K, w, wstride, ca, ra, s);
    return hipGetLastError();
}

bool router_seq_type_ok(int rtype, int K)
{
    if (K <= 0) return false;
    if (rtype == T_F32 || rtype == T_F16) return true;
    if (rtype == T_Q8_0) return K % 32 == 0;
    return (rtype == T_Q4_K || rtype == T_Q6_K) && K % 256 == 0;
}

hipError_t launch_router_rows(int rtype, const uint8_t *rw, uint64_t rstride, int E, int K, float *dst, hipStream_t s)
{
    if (E <= 0 || !router_seq_type_ok(rtype, K) || dst == nullptr) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((K + 255) / 256), (unsigned)E);
    switch (rtype) {
    case T_F32: hipLaunchKernelGGL(k_router_rows_f32<T_F32>, grid, dim3(256), 0, s, rw, rstride, E, K, dst); break;
    case T_F16: hipLaunchKernelGGL(k_router_rows_f32<T_F16>, grid, dim3(256), 0, s, rw, rstride, E, K, dst); break;
    case T_Q8_0: hipLaunchKernelGGL(k_router_rows_f32<T_Q8_0>, grid, dim3(256), 0, s, rw, rstride, E, K, dst); break;
    case T_Q4_K: hipLaunchKernelGGL(k_router_rows_f32<T_Q4_K>, grid, dim3(256), 0, s, rw, rstride, E, K, dst); break;
    default: hipLaunchKernelGGL(k_router_rows_f32<T_Q6_K>, grid, dim3(256), 0, s, rw, rstride, E, K, dst); break;
    }
    return hipGetLastError();
}

template <int DW, int D>
static void seq_launch(const float *x, int T, int K, int E, const float *w, int64_t wstride, float *logits,
                       int64_t ldl, _Float16 *x16, hipStream_t s)
{
    const dim3 grid((unsigned)((T + 15) / 16), (unsigned)((E + 15) / 16));
    hipLaunchKernelGGL((k_router_seq<DW, D>), grid, dim3(256), 0, s, x, T, K, E, w, wstride, logits, ldl, x16);
}

hipError_t launch_router_seq(const float *x, int T, int K, int E, int rtype, const uint8_t *rw, uint64_t rstride,
                             float *wf32, float *logits, int64_t ldl, _Float16 *x16, const RouteArgs *topk,
                             int *tickets, bool *topk_done, hipStream_t s)
{
    if (topk_done) *topk_done = false;
    if (T <= 0 || E <= 0 || E > ROUTE_MAX_E || !router_seq_type_ok(rtype, K)) return hipErrorInvalidValue;
    if (((uintptr_t)x & 3) != 0 || ((uintptr_t)x16 & 1) != 0) return hipErrorInvalidValue;
    const float *w = (const float *)rw;
    int64_t wstride = (int64_t)(rstride / 4);
    const bool f32_direct = rtype == T_F32 && rstride % 4 == 0 && ((uintptr_t)rw & 3) == 0;
    if (!f32_direct) {
        // FP32 copy of the rows as the reference's dequantised router holds them
        if (wf32 == nullptr) return hipErrorInvalidValue;
        const hipError_t er = launch_router_rows(rtype, rw, rstride, E, K, wf32, s);
        if (er != hipSuccess) return er;
        w = wf32;
        wstride = K;
    }
    // 16-byte DMAs need 16-byte aligned rows; 4-byte ones take any float rows
    const bool vec = K % 4 == 0 && wstride % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
                     ((uintptr_t)x16 & 15) == 0;
    // 4 stages (3 chunks in flight, one 133 KB workgroup per CU) while the
    // grid fits one round of the CUs; past that 2 stages, two workgroups per
    // CU in one round (MI355X, T=1024: 26.6 against 36.2 us with 4 stages in
    // two rounds; T=768 25.3 against 34.9)
    const bool deep = (int64_t)((T + 15) / 16) * ((E + 15) / 16) <= device_cu_count();
    RouteArgs none{};
    if (vec && x16 == nullptr && T <= 4) {
        // one token group: fuse top-k when the caller gave a ticket
        const bool fuse = topk != nullptr && tickets != nullptr && topk->logits == logits &&
                          topk->logit_stride == ldl && topk->T == T && topk->E == E;
        const dim3 grid((unsigned)((T + 3) / 4), (unsigned)((E + 3) / 4));
        hipLaunchKernelGGL(k_router_small<4>, grid, dim3(192), 0, s, x, T, K, E, w, wstride, logits, ldl,
                           fuse ? *topk : none, tickets);
        if (fuse && topk_done) *topk_done = true;
    } else if (vec && x16 == nullptr && T <= RSM_MAX_T) {
        const dim3 grid((unsigned)((T + 3) / 4), (unsigned)((E + 15) / 16));
        hipLaunchKernelGGL(k_router_small<16>, grid, dim3(192), 0, s, x, T, K, E, w, wstride, logits, ldl, none,
                           tickets);
    } else if (vec) {
        if (deep) seq_launch<16, 4>(x, T, K, E, w, wstride, logits, ldl, x16, s);
        else seq_launch<16, 2>(x, T, K, E, w, wstride, logits, ldl, x16, s);
    } else {
        seq_launch<4, 2>(x, T, K, E, w, wstride, logits, ldl, x16, s);
    }
    return hipGetLastError();
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
