// moe_grouped.hip -- grouped expert products for many tokens (prefill).
//
// Replaces the reference's per-expert gather -> matmul_quantized_batch x3 ->
// silu_mul -> scatter sequence (src/ds3_engine.c:969-1016,
// metal/matmul_q4k.metal:247-286) with two MFMA kernels over the bucketed
// token lists:
//   gate_up: H[pos][r] = silu(X_e . Wg_e[r]) * (X_e . Wu_e[r])   (fp16 out)
//   down:    Y[pos][j] = H_e[pos] . Wd_e[j]                       (fp16 out)
// where pos runs over expert e's compacted token positions.
//
// Precision: operands are fp16 (x, dequantised weights, h), accumulation is
// fp32 in v_mfma_f32_16x16x32_f16.  Each weight is one fp32-precision FMA on
// its code, rounded once to fp16 (common.h RawUnits::decode_frags).
//
// Structure.  Workgroups are persistent (one per CU, 8 waves) and walk the
// bucketing kernel's run list in an XCD-aware order.  A run is one 64-token
// tile of one expert and a few consecutive 128-row output tiles.  Each wave
// owns 16 output rows (gate_up: the same 16 rows of gate and of up, so
// SwiGLU happens in registers) and streams their quantised blocks straight
// into VGPRs through a ring of register stages, one step ahead of the step
// it decodes, with explicit waits.  Activation rows go to LDS by
// global_load_lds DMA: down's whole tile (64 rows x 768 halves = 96 KiB)
// once per run, so its K loop has no barrier; gate_up's (64 rows x 2048
// halves would be 256 KiB) in 512-wide K chunks through two 64 KiB buffers,
// one barrier per chunk of two K steps.
//
// K order.  Per 256-wide K step, lane group g (lanes 16g..16g+15) decodes
// units g and g+4 of its row (common.h); K-slot q of the step is segment
// q%4 of unit g+4*(q/4), and the activation fragment is read from the same K
// positions (slot_k0), so the MFMA's K order is a permutation shared by both
// operands.
//
// A layout in LDS: step-major, [s][row][512 bytes], 16-byte chunk c of a
// row's slice at 16 * (c ^ (row & 15)): the 16 rows one fragment read
// touches fall on different banks, and one 64-lane DMA fills two rows.
#include "common.h"
#include "launch.h"

#include <type_traits>

namespace ds3k {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int GG_WV = 8;                   // waves per workgroup
constexpr int GG_TILE_N = 16 * GG_WV;      // output rows per n tile (gate_up: of gate and of up)
constexpr int GG_SLICE = 512;              // bytes of one activation row per 256-wide K step
constexpr int GG_TILE_M = 64;              // tokens per bucketing tile (down's token tile)
constexpr int GG_CHUNK_STEPS = 2;          // gate_up: 256-wide K steps per activation chunk
constexpr int GG_CHUNK = GG_TILE_M * GG_SLICE * GG_CHUNK_STEPS;   // bytes of one chunk buffer (64 KiB)
constexpr int GG_DN_MAXK = 1024;           // down: F whose activation rows fit in LDS
constexpr int GG_STAGE = 2048;             // per-wave epilogue staging bytes (gate_up, 4 m blocks)
constexpr int GG_GU_LDS = 2 * GG_CHUNK + GG_WV * GG_STAGE;
constexpr int GG_DN_LDS = GG_TILE_M * GG_SLICE * (GG_DN_MAXK / 256);
constexpr int N_XCD = 8;                   // MI355X: workgroups go round-robin to 8 XCDs
static_assert(GG_GU_LDS <= 163840 && GG_DN_LDS <= 163840, "workgroup LDS exceeds the CU's 160 KiB");

#define DS3_LDS __attribute__((address_space(3)))

// Bytes of one row's quantised block per 256-wide K step.
template <int TYPE> struct GgBlk;
template <> struct GgBlk<T_Q4_K> { static constexpr int BLK = 144; };
template <> struct GgBlk<T_Q6_K> { static constexpr int BLK = 210; };
template <> struct GgBlk<T_Q8_0> { static constexpr int BLK = 272; };

__device__ __forceinline__ const uint8_t *gg_ebase(const uint8_t *base, const uint64_t *table, int e, int which,
                                                   uint64_t rows, uint64_t stride)
{
    return base + (table ? table[3 * e + which] : (uint64_t)e * rows * stride);
}

// 16-byte global -> LDS DMA: lane i writes lds + 16*i.
__device__ __forceinline__ void gg_dma16(const void *src, uint32_t lds)
{
    __builtin_amdgcn_global_load_lds(src, (DS3_LDS void *)(uintptr_t)lds, 16, 0, 0);
}

__device__ __forceinline__ void gg_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait for this wave's DMAs (vmcnt 0: the builtin, so the compiler's own
// wait tracking sees it), then the workgroup barrier.
__device__ __forceinline__ void gg_dma_done()
{
    __builtin_amdgcn_s_waitcnt(0x0F70);     // vmcnt(0), expcnt / lgkmcnt unconstrained
    gg_barrier();
}

// Q4_K blocks load as whole 16-byte vectors when the expert's rows are
// 16-byte aligned (always in GGUF files); Q6_K blocks load their scales and d
// in two loads when every block starts on an even byte (even base and row
// stride: 210-byte blocks then sit at 0 or 2 mod 4); Q8_0 loads dwords.
template <int TYPE>
__device__ __forceinline__ bool gg_aligned(const uint8_t *a, const uint8_t *b, uint64_t stride)
{
    if constexpr (TYPE == T_Q4_K) return ((((uintptr_t)a) | ((uintptr_t)b) | stride) & 15) == 0;
    if constexpr (TYPE == T_Q6_K) return ((((uintptr_t)a) | ((uintptr_t)b) | stride) & 1) == 0;
    return true;
}

// Weight stream: explicit loads and waits.  The weight loads are inline asm
// global loads into native vector registers, and a stage is consumed only
// after an asm s_waitcnt vmcnt(N) that names every register of the stage,
// N being the count of weight loads issued after it.  The compiler cannot
// move either, so the D-stage pipeline stays as written (plain loads let it
// sink the prefetch next to its use and wait for everything each step).
// Loads the compiler issues itself can only be older than a stage's loads or
// add to the younger ones, so vmcnt(N) waits at least for the whole stage.
typedef uint32_t gg_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t gg_u32x3 __attribute__((ext_vector_type(3)));

__device__ __forceinline__ void gg_ldx4(gg_u32x4 &d, const uint8_t *p)
{
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(d) : "v"(p) : "memory");
}
__device__ __forceinline__ void gg_ldx3(gg_u32x3 &d, const uint8_t *p)
{
    asm volatile("global_load_dwordx3 %0, %1, off" : "=v"(d) : "v"(p) : "memory");
}
__device__ __forceinline__ void gg_ldx1(uint32_t &d, const uint8_t *p)
{
    asm volatile("global_load_dword %0, %1, off" : "=v"(d) : "v"(p) : "memory");
}
__device__ __forceinline__ void gg_ldu16(uint32_t &d, const uint8_t *p)
{
    asm volatile("global_load_ushort %0, %1, off" : "=v"(d) : "v"(p) : "memory");
}

// One stage of the weight stream: the raw bytes of this lane's units (g and
// g+4) of one step block, as loaded.
//   Q4_K (AL): header + the two 16-byte units;  (!AL): 5 dwords from the
//     aligned address below each of the three 16-byte fields.
//   Q6_K: per half hv, 3 dwords (from the aligned address below) of each
//     field ql_lo 64hv+8g, ql_hi 64hv+32+8g, qh 128+32hv+8g, scales 192+8hv,
//     and d.
//   Q8_0: per unit g+4hv, the 9 aligned dwords holding its 34-byte block.
template <int TYPE, bool AL> struct GgStage;
template <> struct GgStage<T_Q4_K, true> {
    static constexpr int NLOAD = 3;
    gg_u32x4 h, a, b;
    uint32_t sh;
    __device__ __forceinline__ void issue(const uint8_t *blk, int g)
    {
        gg_ldx4(h, blk);
        gg_ldx4(a, blk + 16 + 16 * g);
        gg_ldx4(b, blk + 16 + 16 * (g + 4));
    }
    template <int N> __device__ __forceinline__ void wait() { asm volatile("s_waitcnt vmcnt(%3)" : "+v"(h), "+v"(a), "+v"(b) : "n"(N)); }
    __device__ __forceinline__ void to_raw(RawUnits<T_Q4_K> &r) const
    {
        r.hdr = make_uint4(h.x, h.y, h.z, h.w);
        r.q0 = make_uint4(a.x, a.y, a.z, a.w);
        r.q1 = make_uint4(b.x, b.y, b.z, b.w);
    }
};
template <> struct GgStage<T_Q4_K, false> {
    static constexpr int NLOAD = 6;
    gg_u32x4 v[3];
    uint32_t e[3];
    uint32_t sh;
    __device__ __forceinline__ void issue(const uint8_t *blk, int g)
    {
        sh = (uint32_t)((uintptr_t)blk & 3);
        const uint8_t *pp[3] = { blk, blk + 16 + 16 * g, blk + 16 + 16 * (g + 4) };
#pragma unroll
        for (int f = 0; f < 3; f++) {
            const uint8_t *a = (const uint8_t *)((uintptr_t)pp[f] & ~(uintptr_t)3);
            gg_ldx4(v[f], a);
            gg_ldx1(e[f], a + 16);
        }
    }
    template <int N> __device__ __forceinline__ void wait()
    {
        asm volatile("s_waitcnt vmcnt(%6)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(e[0]), "+v"(e[1]), "+v"(e[2])
                     : "n"(N));
    }
    __device__ __forceinline__ void to_raw(RawUnits<T_Q4_K> &r) const
    {
        uint32_t w[3][4];
#pragma unroll
        for (int f = 0; f < 3; f++) {
            const uint32_t d[5] = { v[f].x, v[f].y, v[f].z, v[f].w, e[f] };
#pragma unroll
            for (int i = 0; i < 4; i++) w[f][i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
        }
        r.hdr = make_uint4(w[0][0], w[0][1], w[0][2], w[0][3]);
        r.q0 = make_uint4(w[1][0], w[1][1], w[1][2], w[1][3]);
        r.q1 = make_uint4(w[2][0], w[2][1], w[2][2], w[2][3]);
    }
};
// Q6_K, blocks on even bytes: the two scale windows and d come from one
// 16-byte load at the aligned address below the scales (offset 192) and one
// dword at offset 208 from it, which holds d (block offset sh is 0 or 2) and
// reads no further past the block than the 12-byte windows do.
template <> struct GgStage<T_Q6_K, true> {
    static constexpr int NLOAD = 8;
    gg_u32x3 f[2][3];
    gg_u32x4 sc;
    uint32_t dd, sh;
    __device__ __forceinline__ void issue(const uint8_t *blk, int g)
    {
        const uint8_t *b4 = (const uint8_t *)((uintptr_t)blk & ~(uintptr_t)3);
        sh = (uint32_t)((uintptr_t)blk & 3);
#pragma unroll
        for (int hv = 0; hv < 2; hv++) {
            const int off[3] = { 64 * hv + 8 * g, 64 * hv + 32 + 8 * g, 128 + 32 * hv + 8 * g };
#pragma unroll
            for (int fi = 0; fi < 3; fi++) gg_ldx3(f[hv][fi], b4 + off[fi]);
        }
        gg_ldx4(sc, b4 + 192);
        gg_ldx1(dd, b4 + 208);
    }
    template <int N> __device__ __forceinline__ void wait()
    {
        asm volatile("s_waitcnt vmcnt(%8)" : "+v"(f[0][0]), "+v"(f[0][1]), "+v"(f[0][2]), "+v"(f[1][0]), "+v"(f[1][1]),
                     "+v"(f[1][2]), "+v"(sc), "+v"(dd) : "n"(N));
    }
    __device__ __forceinline__ void to_raw(RawUnits<T_Q6_K> &r) const
    {
#pragma unroll
        for (int hv = 0; hv < 2; hv++)
#pragma unroll
            for (int fi = 0; fi < 3; fi++) {
                r.f[hv][fi][0] = f[hv][fi].x;
                r.f[hv][fi][1] = f[hv][fi].y;
                r.f[hv][fi][2] = f[hv][fi].z;
            }
        // the 12-byte scale windows at 192 and 200 from b4
        r.f[0][3][0] = sc.x; r.f[0][3][1] = sc.y; r.f[0][3][2] = sc.z;
        r.f[1][3][0] = sc.z; r.f[1][3][1] = sc.w; r.f[1][3][2] = dd;
        r.dw = (dd >> (8 * sh)) & 0xffffu;
        r.sh = sh;
    }
};
template <bool AL> struct GgStage<T_Q6_K, AL> {
    static constexpr int NLOAD = 9;
    gg_u32x3 f[2][4];
    uint32_t dw, sh;
    __device__ __forceinline__ void issue(const uint8_t *blk, int g)
    {
        const uint8_t *b4 = (const uint8_t *)((uintptr_t)blk & ~(uintptr_t)3);
        sh = (uint32_t)((uintptr_t)blk & 3);
#pragma unroll
        for (int hv = 0; hv < 2; hv++) {
            const int off[4] = { 64 * hv + 8 * g, 64 * hv + 32 + 8 * g, 128 + 32 * hv + 8 * g, 192 + 8 * hv };
#pragma unroll
            for (int fi = 0; fi < 4; fi++) gg_ldx3(f[hv][fi], b4 + off[fi]);
        }
        gg_ldu16(dw, blk + 208);
    }
    template <int N> __device__ __forceinline__ void wait()
    {
        asm volatile("s_waitcnt vmcnt(%9)" : "+v"(f[0][0]), "+v"(f[0][1]), "+v"(f[0][2]), "+v"(f[0][3]), "+v"(f[1][0]),
                     "+v"(f[1][1]), "+v"(f[1][2]), "+v"(f[1][3]), "+v"(dw) : "n"(N));
    }
    __device__ __forceinline__ void to_raw(RawUnits<T_Q6_K> &r) const
    {
#pragma unroll
        for (int hv = 0; hv < 2; hv++)
#pragma unroll
            for (int fi = 0; fi < 4; fi++) {
                r.f[hv][fi][0] = f[hv][fi].x;
                r.f[hv][fi][1] = f[hv][fi].y;
                r.f[hv][fi][2] = f[hv][fi].z;
            }
        r.dw = dw & 0xffffu;
        r.sh = sh;
    }
};
template <bool AL> struct GgStage<T_Q8_0, AL> {
    static constexpr int NLOAD = 6;
    gg_u32x4 v[2][2];
    uint32_t e[2];
    uint32_t sh[2];
    __device__ __forceinline__ void issue(const uint8_t *blk, int g)
    {
#pragma unroll
        for (int hv = 0; hv < 2; hv++) {
            const uintptr_t o = (uintptr_t)blk + (uintptr_t)(34 * (g + 4 * hv));
            sh[hv] = (uint32_t)(o & 3);
            const uint8_t *p = (const uint8_t *)(o & ~(uintptr_t)3);
            gg_ldx4(v[hv][0], p);
            gg_ldx4(v[hv][1], p + 16);
            gg_ldx1(e[hv], p + 32);
        }
    }
    template <int N> __device__ __forceinline__ void wait()
    {
        asm volatile("s_waitcnt vmcnt(%6)" : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[1][0]), "+v"(v[1][1]), "+v"(e[0]),
                     "+v"(e[1]) : "n"(N));
    }
    __device__ __forceinline__ void to_raw(RawUnits<T_Q8_0> &r) const
    {
#pragma unroll
        for (int hv = 0; hv < 2; hv++) {
            const uint32_t d[9] = { v[hv][0].x, v[hv][0].y, v[hv][0].z, v[hv][0].w,
                                    v[hv][1].x, v[hv][1].y, v[hv][1].z, v[hv][1].w, e[hv] };
#pragma unroll
            for (int i = 0; i < 9; i++) r.q[hv][i] = d[i];
            r.sh[hv] = sh[hv];
        }
    }
};

// Activation fragments of K-slots q0 and q0+1 for MB m blocks: lane (g, m)
// reads row 16mb + m at its slot's chunk.  gg_afrag_issue issues the reads;
// gg_afrag_wait waits for all of them, naming every result so nothing reads
// them early.  In between, the weight fragments are decoded, which hides the
// LDS latency.
template <int MB>
__device__ __forceinline__ void gg_afrag_issue(uint32_t a0, uint32_t a1, half8 (&af)[2][MB])
{
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[0][mb]) : "v"(a0), "i"(16 * GG_SLICE * mb));
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[1][mb]) : "v"(a1), "i"(16 * GG_SLICE * mb));
    }
}

template <int MB>
__device__ __forceinline__ void gg_afrag_wait(half8 (&af)[2][MB])
{
    if constexpr (MB == 1)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(af[0][0]), "+v"(af[1][0]));
    else if constexpr (MB == 2)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(af[0][0]), "+v"(af[1][0]), "+v"(af[0][1]), "+v"(af[1][1]));
    else if constexpr (MB == 3)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(af[0][0]), "+v"(af[1][0]), "+v"(af[0][1]), "+v"(af[1][1]),
                     "+v"(af[0][2]), "+v"(af[1][2]));
    else
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(af[0][0]), "+v"(af[1][0]), "+v"(af[0][1]), "+v"(af[1][1]),
                     "+v"(af[0][2]), "+v"(af[1][2]), "+v"(af[0][3]), "+v"(af[1][3]));
}

// One 256-wide K step for NB column blocks of 16 rows (gate_up: NB = 2,
// gate and up of the same rows; down: NB = 1); sb = LDS byte address of the
// step's activation slice, lofs[q] = this lane's byte offset of K-slot q in
// it.
template <int TYPE, int NB, int MB>
__device__ __forceinline__ void gg_step(const RawUnits<TYPE> (&raw)[NB], uint32_t sb, const uint32_t (&lofs)[8],
                                        int g, floatx4 (&acc)[MB][NB])
{
#pragma unroll
    for (int hv = 0; hv < 2; hv++) {
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            half8 af[2][MB];
            gg_afrag_issue<MB>(sb + lofs[4 * hv + 2 * pp], sb + lofs[4 * hv + 2 * pp + 1], af);
            // only the two fragments this half step feeds stay live (the
            // compiler drops the other two and shares the scale set-up)
            half8 bq[NB][2];
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                half8 fr[4];
                raw[nb].decode_frags(hv, g, fr);
                bq[nb][0] = fr[2 * pp];
                bq[nb][1] = fr[2 * pp + 1];
            }
            gg_afrag_wait<MB>(af);
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[p][mb], bq[nb][p], acc[mb][nb], 0,
                                                                              0, 0);
        }
    }
}

// A K loop leaves D - 1 weight stages loading past its last step (every
// stage is issued unconditionally).  Wait for them before the loop returns,
// naming every register of every stage, so no later code can be given a
// register that a late load still writes.
template <int D, int NB, class St>
__device__ __forceinline__ void gg_ring_drain(St (&ring)[D][NB])
{
#pragma unroll
    for (int d = 0; d < D; d++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) ring[d][nb].template wait<0>();
}

// The K loop of a run: U = nnt * S steps (n tile t = u / S, K step u % S),
// weights of step u + D - 1 loaded while step u is decoded; after the last K
// step of an n tile the epilogue stores it.  rows[nb]: this lane's weight row
// in the run's first n tile; tstride: bytes between the same row of
// consecutive n tiles.
template <int TYPE, bool AL, int NB, int MB, int D, class Epi>
__device__ __forceinline__ void gg_run(const uint8_t *const (&rows)[NB], uint64_t tstride, int S, int nnt,
                                       uint32_t a_lds, uint32_t step_bytes, const uint32_t (&lofs)[8], int g,
                                       const Epi &epi)
{
    constexpr int BLK = GgBlk<TYPE>::BLK;
    const int U = nnt * S;
    floatx4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };
    using St = GgStage<TYPE, AL>;
    St ring[D][NB];
    const uint8_t *wp[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) wp[nb] = rows[nb];
    int ls = 0, left = U;                               // K step and count of the loads still to come
    // Every stage is issued unconditionally, so the same D-1 stages are in
    // flight behind each stage on every path; past the run's last step the
    // pointer stays on the last block (those loads re-read it from L2 and are
    // never decoded).
    auto issue = [&](St(&dst)[NB]) {
#pragma unroll
        for (int nb = 0; nb < NB; nb++) dst[nb].issue(wp[nb], g);
        if (--left > 0) {
            const int64_t adv = ++ls == S ? (int64_t)tstride - (int64_t)(S - 1) * BLK : (int64_t)BLK;
            if (ls == S) ls = 0;
#pragma unroll
            for (int nb = 0; nb < NB; nb++) wp[nb] += adv;
        }
    };
#pragma unroll
    for (int i = 0; i < D - 1; i++) issue(ring[i]);
    int cs = 0, ct = 0;                                 // K step and n tile of the step computed next
    for (int u0 = 0; u0 < U; u0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            issue(ring[(d + D - 1) % D]);
            // stage d was issued D-1 stages before the ones now in flight
            constexpr int NV = (D - 1) * NB * St::NLOAD;
            static_assert(NV <= 63, "vmcnt field holds 0..63");
#pragma unroll
            for (int nb = 0; nb < NB; nb++) ring[d][nb].template wait<NV>();
            if (u0 + d < U) {
                RawUnits<TYPE> raw[NB];
#pragma unroll
                for (int nb = 0; nb < NB; nb++) ring[d][nb].to_raw(raw[nb]);
                gg_step<TYPE, NB, MB>(raw, a_lds + (uint32_t)cs * step_bytes, lofs, g, acc);
                if (++cs == S) {
                    epi.template store<MB>(acc, ct);
#pragma unroll
                    for (int i = 0; i < MB; i++)
#pragma unroll
                        for (int j = 0; j < NB; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };
                    cs = 0;
                    ct++;
                }
            }
        }
    }
    gg_ring_drain<D, NB>(ring);
}

// gate_up's K loop: activation rows stream through two LDS chunk buffers of
// GG_CHUNK_STEPS = 2 K steps each (chunk c of the run = n tile c / (S / 2), K
// steps 2 * (c % (S / 2)) .. +1, in buffer c & 1), weights through a ring of
// D register stages, D - 1 steps ahead.  Issue order, every item
// unconditional so the wait counts are static:
//   chunk c:  [A(c+1) DMAs]  step 2c: [W(2c+D-1)] wait W(2c) [compute]
//                            step 2c+1: [W(2c+D)] wait W(2c+1) [compute]
//             wait A(c+1), barrier, then A(c+2) into buffer c & 1
// a_src(c, dst): this wave's NA DMAs of chunk c (clamped to the run's last
// chunk) into LDS buffer address dst.
template <int TYPE, bool AL, int MB, int NA, int D, class ASrc, class Epi>
__device__ __forceinline__ void gg_run_chunked(const uint8_t *const (&rows)[2], uint64_t tstride, int S, int nnt,
                                               uint32_t a_lds, const uint32_t (&lofs)[8], int g, const ASrc &a_src,
                                               const Epi &epi)
{
    constexpr int NB = 2, BLK = GgBlk<TYPE>::BLK;
    using St = GgStage<TYPE, AL>;
    constexpr int NW = NB * St::NLOAD;
    static_assert(NA + (D - 1) * NW <= 63, "vmcnt field holds 0..63");
    // one loop iteration is D steps: whole chunks and one turn of the ring,
    // so both stay in step across n tiles (K a multiple of 256 * D)
    static_assert(D % GG_CHUNK_STEPS == 0, "the chunked K loop turns the weight ring once per D / 2 chunks");
    constexpr int UNR = D;
    const int U = nnt * S;
    floatx4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };
    St ring[D][NB];
    const uint8_t *wp[NB] = { rows[0], rows[1] };
    int ls = 0, left = U;
    auto issue = [&](St(&dst)[NB]) {
#pragma unroll
        for (int nb = 0; nb < NB; nb++) dst[nb].issue(wp[nb], g);
        if (--left > 0) {
            const int64_t adv = ++ls == S ? (int64_t)tstride - (int64_t)(S - 1) * BLK : (int64_t)BLK;
            if (ls == S) ls = 0;
#pragma unroll
            for (int nb = 0; nb < NB; nb++) wp[nb] += adv;
        }
    };
    auto step = [&](St(&st)[NB], uint32_t sb) {
        RawUnits<TYPE> raw[NB];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) st[nb].to_raw(raw[nb]);
        gg_step<TYPE, NB, MB>(raw, sb, lofs, g, acc);
    };
    // chunk 0 and the first D-1 weight stages; everything landed, then the barrier
    a_src(0, a_lds);
#pragma unroll
    for (int i = 0; i < D - 1; i++) issue(ring[i]);
    __builtin_amdgcn_s_waitcnt(0x0F70);               // vmcnt(0)
    gg_barrier();
    a_src(1, a_lds + GG_CHUNK);
    // n tiles outside, chunks inside: the epilogue (SwiGLU, stores) sits
    // after the chunk loop, where the compiler cannot hoist its math into
    // every step.  Each loop iteration is UNR steps (whole chunks and whole
    // turns of the ring); chunks run on across n tiles.
    const int cpt = S / GG_CHUNK_STEPS;                   // chunks per n tile
    int c = 0;                                            // chunk index within the run
    for (int t = 0; t < nnt; t++) {
        for (int i0 = 0; i0 < cpt * GG_CHUNK_STEPS; i0 += UNR) {
#pragma unroll
            for (int d = 0; d < UNR; d++) {
                issue(ring[(d + D - 1) % D]);
                // Loads in flight behind W(u): the D-1 later stages, and
                // A(c'+1) for every chunk c' whose DMAs went out between them
                // (A(c'+1) follows W(2c'+D-2)).  At least one such A for the
                // first step of a chunk (one in the first chunk, two later for
                // D = 4: counting fewer only waits longer, for a chunk already
                // landed), one for the second step if D >= 3.
                constexpr int NEVEN = NA + (D - 1) * NW, NODD = (D >= 3 ? NA : 0) + (D - 1) * NW;
#pragma unroll
                for (int nb = 0; nb < NB; nb++) {
                    if ((d & 1) == 0) ring[d % D][nb].template wait<NEVEN>();    // folds: d is unrolled
                    else ring[d % D][nb].template wait<NODD>();
                }
                step(ring[d % D], a_lds + (uint32_t)(c & 1) * GG_CHUNK + (uint32_t)(d & 1) * (GG_TILE_M * GG_SLICE));
                if (d & 1) {
                    // end of chunk c: A(c+1) went out before W(2c+D-1) and W(2c+D)
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NW) : "memory");
                    gg_barrier();
                    a_src(c + 2, a_lds + (uint32_t)(c & 1) * GG_CHUNK);
                    c++;
                }
            }
        }
        epi.template store<MB>(acc, t);
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < NB; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };
    }
    gg_ring_drain<D, NB>(ring);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");     // the last chunk DMA (a_src) has landed too
}

// This lane's byte offsets of the 8 K-slots in a step's activation slice.
template <int TYPE>
__device__ __forceinline__ void gg_lofs(int lane, uint32_t (&lofs)[8])
{
    const int g = lane >> 4, m = lane & 15;
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const uint32_t c = (uint32_t)slot_k0<TYPE>(0, g, q) / 8u;
        lofs[q] = (uint32_t)(m * GG_SLICE) + 16u * (c ^ (uint32_t)m);
    }
}

// Activation rows of a run into LDS: rows 0 .. 16*MB-1 of the tile (rows at
// or past mrows repeat row 0), K = 256*S halves each, step-major.  Row r's
// source is src_row(r); DMA instruction i (of S * 8 * MB) fills row pair
// 2 * (i % (8*MB)) of step i / (8*MB); wave w issues i = w, w + 8, ...
template <int MB, class SrcRow>
__device__ __forceinline__ void gg_fill_a(uint32_t a_lds, int rows_alloc, int S, int mrows, int wave, int lane,
                                          const SrcRow &src_row)
{
    const _Float16 *src[MB];
#pragma unroll
    for (int kk = 0; kk < MB; kk++) {
        const int row = 2 * (wave + GG_WV * kk) + (lane >> 5);
        const int chunk = (lane & 31) ^ (row & 15);
        src[kk] = src_row(row < mrows ? row : 0) + 8 * chunk;
    }
    const uint32_t sbytes = (uint32_t)(rows_alloc * GG_SLICE);
    for (int s = 0; s < S; s++)
#pragma unroll
        for (int kk = 0; kk < MB; kk++)
            gg_dma16(src[kk] + 256 * s, a_lds + (uint32_t)s * sbytes + (uint32_t)(2 * (wave + GG_WV * kk) * GG_SLICE));
}

// Persistent schedule over the bucketing kernel's run list (heaviest runs
// first): round k of the grid (gridDim.x a multiple of 8; workgroup w sits on
// XCD w % 8) takes list entries k*G .. k*G+G-1, consecutive entries on the
// same XCD, so token tiles of one expert (adjacent in the list) stream the
// same weights through one L2 at the same time.  Odd rounds go through their
// entries in reverse, so the workgroup that took the heaviest run of one
// round takes the lightest of the next.
__device__ __forceinline__ int gg_list_index(int k)
{
    const int G = (int)gridDim.x, w = (int)blockIdx.x;
    const int s = (G / N_XCD) * (w % N_XCD) + w / N_XCD;
    return k * G + ((k & 1) ? G - 1 - s : s);
}

// gate_up epilogue: h = silu(gate) * up as fp16, staged through a per-wave
// LDS patch so each lane stores 4 consecutive columns (8 bytes) of a token
// row instead of 4 scattered halves.
struct GgEpiGateUp {
    _Float16 *h16;
    int F, row0, mrows, nt0, wave, lane;
    uint32_t stage;                 // this wave's LDS staging patch
    template <int MB>
    __device__ __forceinline__ void store(const floatx4 (&acc)[MB][2], int t) const
    {
        const int g = lane >> 4, m = lane & 15;
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const _Float16 v = (_Float16)swiglu(acc[mb][0][j], acc[mb][1][j]);
                const uint32_t a = stage + (uint32_t)(2 * (mb * 256 + (4 * g + j) * 16 + m));
                asm volatile("ds_write_b16 %0, %1" ::"v"(a), "v"(v) : "memory");
            }
        const int tok = lane >> 2, cq = lane & 3;
        const int col = (nt0 + t) * GG_TILE_N + 16 * wave + 4 * cq;
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            uint2 v;
            asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                         : "=v"(v)
                         : "v"(stage + (uint32_t)(2 * (mb * 256 + tok * 16 + 4 * cq)))
                         : "memory");
            const int mr = 16 * mb + tok;
            if (mr < mrows) *(uint2 *)(h16 + (int64_t)(row0 + mr) * F + col) = v;
        }
    }
};

// down epilogue: y rows in fp16, rounded once from the fp32 accumulators
// (each store instruction writes 4 rows x 16 consecutive columns).
struct GgEpiDown {
    _Float16 *y;
    int N, row0, mrows, nt0, wave, lane;
    template <int MB>
    __device__ __forceinline__ void store(const floatx4 (&acc)[MB][1], int t) const
    {
        const int g = lane >> 4, m = lane & 15;
        const int col = (nt0 + t) * GG_TILE_N + 16 * wave + m;
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int mr = 16 * mb + 4 * g + j;
                if (mr < mrows) y[(int64_t)(row0 + mr) * N + col] = (_Float16)acc[mb][0][j];
            }
    }
};

// Plain-product epilogue (dense C = A W^T on the gate_up kernel): the two
// row sets of a run are the two halves of W, rows n and n + half; C rows in
// fp32 (each store instruction writes 4 rows x 16 consecutive columns).
struct GgEpiPlain {
    float *c;
    int N, half, row0, mrows, nt0, wave, lane;
    template <int MB>
    __device__ __forceinline__ void store(const floatx4 (&acc)[MB][2], int t) const
    {
        const int g = lane >> 4, m = lane & 15;
        const int col = (nt0 + t) * GG_TILE_N + 16 * wave + m;
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int mr = 16 * mb + 4 * g + j;
                if (mr < mrows) {
                    float *row = c + (int64_t)(row0 + mr) * N;
                    row[col] = acc[mb][0][j];
                    row[half + col] = acc[mb][1][j];
                }
            }
    }
};

template <int TYPE, bool AL, int NB, int D, class Epi>
__device__ __forceinline__ void gg_run_mb(int mb, const uint8_t *const (&rows)[NB], uint64_t tstride, int S, int nnt,
                                          uint32_t a_lds, uint32_t step_bytes, const uint32_t (&lofs)[8], int g,
                                          const Epi &epi)
{
    switch (mb) {
    case 1: gg_run<TYPE, AL, NB, 1, D>(rows, tstride, S, nnt, a_lds, step_bytes, lofs, g, epi); break;
    case 2: gg_run<TYPE, AL, NB, 2, D>(rows, tstride, S, nnt, a_lds, step_bytes, lofs, g, epi); break;
    case 3:
        if constexpr (NB == 1) gg_run<TYPE, AL, NB, 3, D>(rows, tstride, S, nnt, a_lds, step_bytes, lofs, g, epi);
        break;
    default:
        if constexpr (NB == 1) gg_run<TYPE, AL, NB, 4, D>(rows, tstride, S, nnt, a_lds, step_bytes, lofs, g, epi);
        break;
    }
}

#ifndef DS3_GG_DEPTH
#define DS3_GG_DEPTH 2              // down: register stages of the weight stream (D - 1 steps ahead)
#endif
#ifndef DS3_GU_DEPTH
#define DS3_GU_DEPTH 2              // gate_up: register stages of the weight stream
#endif

// A's DMAs of K chunk c (clamped to the run's last) into the buffer at dst:
// rows 0 .. 16*MB-1 of the tile (rows at or past mrows repeat row 0), two
// step slices; instruction i (of 16 * MB) fills row pair i % (8*MB) of slice
// i / (8*MB); wave w issues i = w, w + 8, ... (2 * MB of them).
template <int MB>
struct GgAChunks {
    const _Float16 *src[MB];        // this lane's source chunk of its row pairs, K step 0
    int S, nch, wave;
    __device__ __forceinline__ void operator()(int c, uint32_t dst) const
    {
        const int cc = c < nch ? c : nch - 1;
        const int k0 = 256 * GG_CHUNK_STEPS * (cc % (S / GG_CHUNK_STEPS));
#pragma unroll
        for (int sl = 0; sl < GG_CHUNK_STEPS; sl++)
#pragma unroll
            for (int kk = 0; kk < MB; kk++)
                gg_dma16(src[kk] + k0 + 256 * sl,
                         dst + (uint32_t)(sl * GG_TILE_M * GG_SLICE + 2 * (wave + GG_WV * kk) * GG_SLICE));
    }
};

template <int TYPE, bool AL, int MB, class Epi>
__device__ __forceinline__ void gg_gate_up_run(const _Float16 *x16, int K, const int32_t *ids, int mrows,
                                               const uint8_t *const (&rows)[2], uint64_t tstride, int nnt,
                                               uint32_t a_lds, const uint32_t (&lofs)[8], int wave, int lane,
                                               const Epi &epi)
{
    const int S = K / 256;
    GgAChunks<MB> as;
    as.S = S;
    as.nch = nnt * S / GG_CHUNK_STEPS;
    as.wave = wave;
#pragma unroll
    for (int kk = 0; kk < MB; kk++) {
        const int row = 2 * (wave + GG_WV * kk) + (lane >> 5);
        const int chunk = (lane & 31) ^ (row & 15);
        as.src[kk] = x16 + (int64_t)ids[row < mrows ? row : 0] * K + 8 * chunk;
    }
    gg_run_chunked<TYPE, AL, MB, GG_CHUNK_STEPS * MB, DS3_GU_DEPTH>(rows, tstride, S, nnt, a_lds, lofs, lane >> 4, as,
                                                                   epi);
}

// PLAIN: a dense product C[M][2F] = A W^T instead (one expert, W's rows
// [0, F) in the gate slot and [F, 2F) in the up slot), fp32 C in place of h.
template <int TYPE, bool PLAIN = false>
__global__ void __launch_bounds__(64 * GG_WV)
k_grouped_gate_up(const _Float16 *__restrict__ x16, int K, ExpertWeights ew, int F, BucketOut b,
                  _Float16 *__restrict__ h16, int ntb, float *__restrict__ c = nullptr)
{
    __shared__ __attribute__((aligned(16))) uint8_t smem[GG_GU_LDS];
    const int n_nt = F / GG_TILE_N;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t a_lds = (uint32_t)(uintptr_t)(DS3_LDS void *)smem;
    const uint32_t stage = a_lds + (uint32_t)(2 * GG_CHUNK + wave * GG_STAGE);
    uint32_t lofs[8];
    gg_lofs<TYPE>(lane, lofs);
    // the run count and the first run's descriptor in one round trip; each
    // later descriptor is loaded while the run before it computes
    const int n_runs = b.n_runs[0], cap = b.max_tiles * b.rpi_gu;
    int i = gg_list_index(0);
    int2 d = b.desc_gu[min(i, cap - 1)];
    for (int k = 0; i < n_runs; k++) {                      // uniform over the workgroup
        const int e = d.y >> 16, mrows = (d.y >> 8) & 255, j = d.y & 255, row0 = d.x;
        const int mblocks = (mrows + 15) / 16;
        const int nt0 = j * ntb, nnt = min(ntb, n_nt - nt0);
        // every wave's DMAs of the previous run have landed and its reads of
        // the buffers are done before this run's DMAs overwrite them
        gg_dma_done();
        i = gg_list_index(k + 1);
        d = b.desc_gu[min(i, cap - 1)];
        const int32_t *ids = b.ids + row0;
        const uint8_t *wg = gg_ebase(ew.gate, ew.table, e, 0, (uint64_t)F, ew.gate_stride);
        const uint8_t *wu = gg_ebase(ew.up, ew.table, e, 1, (uint64_t)F, ew.up_stride);
        const size_t r0 = (size_t)nt0 * GG_TILE_N + 16 * wave + (lane & 15);
        const uint8_t *const rows[2] = { wg + r0 * ew.gate_stride, wu + r0 * ew.up_stride };
        const uint64_t tstride = (uint64_t)GG_TILE_N * ew.gate_stride;    // gate and up strides are equal
        const bool al = gg_aligned<TYPE>(wg, wu, ew.gate_stride);
        using Epi = std::conditional_t<PLAIN, GgEpiPlain, GgEpiGateUp>;
        Epi epi;
        if constexpr (PLAIN) epi = GgEpiPlain{ c, 2 * F, F, row0, mrows, nt0, wave, lane };
        else epi = GgEpiGateUp{ h16, F, row0, mrows, nt0, wave, lane, stage };
#define DS3_GU_CASE(MBV)                                                                                      \
    if (al) gg_gate_up_run<TYPE, true, MBV>(x16, K, ids, mrows, rows, tstride, nnt, a_lds, lofs, wave, lane, epi); \
    else gg_gate_up_run<TYPE, false, MBV>(x16, K, ids, mrows, rows, tstride, nnt, a_lds, lofs, wave, lane, epi);
        switch (mblocks) {
        case 1: DS3_GU_CASE(1) break;
        case 2: DS3_GU_CASE(2) break;
        case 3: DS3_GU_CASE(3) break;
        default: DS3_GU_CASE(4) break;
        }
#undef DS3_GU_CASE
    }
}

template <int TYPE>
__global__ void __launch_bounds__(64 * GG_WV)
k_grouped_down(const _Float16 *__restrict__ h16, int F, ExpertWeights ew, int N, BucketOut b,
               _Float16 *__restrict__ y, int ntb)
{
    __shared__ __attribute__((aligned(16))) uint8_t smem[GG_DN_LDS];
    const int n_nt = N / GG_TILE_N;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), g = lane >> 4;
    const int S = F / 256;
    const uint32_t a_lds = (uint32_t)(uintptr_t)(DS3_LDS void *)smem;
    const uint32_t step_bytes = (uint32_t)(GG_TILE_M * GG_SLICE);
    uint32_t lofs[8];
    gg_lofs<TYPE>(lane, lofs);
    // the run count and the first run's descriptor in one round trip; each
    // later descriptor is loaded while the run before it computes
    const int n_runs = b.n_runs[1], cap = b.max_tiles * b.rpi_dn;
    int i = gg_list_index(0);
    int2 d = b.desc_dn[min(i, cap - 1)];
    for (int k = 0; i < n_runs; k++) {                      // uniform over the workgroup
        const int e = d.y >> 16, mrows = (d.y >> 8) & 255, run = d.y & 255, row0 = d.x;
        const int mblocks = (mrows + 15) / 16;
        const int nt0 = run * ntb, nnt = min(ntb, n_nt - nt0);
        gg_barrier();
        auto src_row = [&](int r) { return h16 + (int64_t)(row0 + r) * F; };
        switch (mblocks) {
        case 1: gg_fill_a<1>(a_lds, GG_TILE_M, S, mrows, wave, lane, src_row); break;
        case 2: gg_fill_a<2>(a_lds, GG_TILE_M, S, mrows, wave, lane, src_row); break;
        case 3: gg_fill_a<3>(a_lds, GG_TILE_M, S, mrows, wave, lane, src_row); break;
        default: gg_fill_a<4>(a_lds, GG_TILE_M, S, mrows, wave, lane, src_row); break;
        }
        const uint8_t *wd = gg_ebase(ew.down, ew.table, e, 2, (uint64_t)N, ew.down_stride);
        const uint8_t *const rows[1] = { wd + ((size_t)nt0 * GG_TILE_N + 16 * wave + (lane & 15)) * ew.down_stride };
        const uint64_t tstride = (uint64_t)GG_TILE_N * ew.down_stride;
        const GgEpiDown epi{ y, N, row0, mrows, nt0, wave, lane };
        gg_dma_done();
        i = gg_list_index(k + 1);
        d = b.desc_dn[min(i, cap - 1)];
        if (gg_aligned<TYPE>(wd, wd, ew.down_stride))
            gg_run_mb<TYPE, true, 1, DS3_GG_DEPTH>(mblocks, rows, tstride, S, nnt, a_lds, step_bytes, lofs, g, epi);
        else
            gg_run_mb<TYPE, false, 1, DS3_GG_DEPTH>(mblocks, rows, tstride, S, nnt, a_lds, step_bytes, lofs, g, epi);
    }
}

// Dense C[M][N] = A[M][K] W[N][K]^T on the gate_up kernel: the bucketing
// lists of one expert holding every row of A (b), x16 = A in fp16.
template <int TV>
static hipError_t dense_t(const _Float16 *x16, int K, const ExpertWeights &ew, int N, const BucketOut &b, float *c,
                          hipStream_t s);

bool grouped_type_ok(int type, int K)
{
    if (K <= 0 || K % 256 != 0) return false;
    return type == T_Q4_K || type == T_Q6_K || type == T_Q8_0;
}

bool grouped_shape_ok(int n_embd, int n_ff)
{
    return n_embd % (256 * DS3_GU_DEPTH) == 0 && n_ff % GG_TILE_N == 0 && n_embd % GG_TILE_N == 0 &&
           n_ff <= GG_DN_MAXK;
}

// n tiles per down run (tuning knob).
#ifndef DS3_DN_NTB
#define DS3_DN_NTB 8
#endif

int device_cu_count()
{
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    return n_cu;
}

// n tiles per gate_up run: 3 while the call's runs fit one round of the
// persistent grid, else 2, whose shorter runs balance the rounds (MI355X,
// Qwen3-30B-A3B layer: T=512 164.6 us per step with 3 against 179.0 with 2;
// T=2048 Zipf 402.6 with 2 against 413 with 3).  The work items are
// estimated from the call's S slots and E experts as S / 64 + E / 2 (every
// expert's partial last tile counted as half an item on average).
void grouped_runs_per_tile(int n_embd, int n_ff, int S, int E, int &rpi_gu, int &rpi_dn)
{
    const int n_nt = n_ff / GG_TILE_N, items = S / GG_TILE_M + E / 2;
    const int ntb = (int64_t)items * ((n_nt + 2) / 3) <= device_cu_count() ? 3 : 2;
    rpi_gu = (n_nt + ntb - 1) / ntb;
    rpi_dn = (n_embd / GG_TILE_N + DS3_DN_NTB - 1) / DS3_DN_NTB;
}

// Persistent grid: one workgroup per CU (a multiple of 8), or fewer when the
// run list cannot be that long.
static unsigned gg_grid(int max_runs)
{
    const int n_cu = device_cu_count();
    const int g = (n_cu + N_XCD - 1) / N_XCD * N_XCD, need = (max_runs + N_XCD - 1) / N_XCD * N_XCD;
    return (unsigned)(need < g ? (need > 0 ? need : N_XCD) : g);
}

template <int TV>
static hipError_t gate_up_t(const _Float16 *x16, int K, const ExpertWeights &ew, int F, const BucketOut &b,
                            _Float16 *h16, hipStream_t s)
{
    const unsigned grid = gg_grid(b.max_tiles * b.rpi_gu);
    const int n_nt = F / GG_TILE_N, ntb = (n_nt + b.rpi_gu - 1) / b.rpi_gu;     // n tiles per run
    hipLaunchKernelGGL((k_grouped_gate_up<TV>), dim3(grid), dim3(64 * GG_WV), 0, s, x16, K, ew, F, b, h16, ntb);
    return hipGetLastError();
}

template <int TV>
static hipError_t down_t(const _Float16 *h16, int F, const ExpertWeights &ew, int N, const BucketOut &b,
                         _Float16 *y, hipStream_t s)
{
    const unsigned grid = gg_grid(b.max_tiles * b.rpi_dn);
    hipLaunchKernelGGL((k_grouped_down<TV>), dim3(grid), dim3(64 * GG_WV), 0, s, h16, F, ew, N, b, y,
                       DS3_DN_NTB);
    return hipGetLastError();
}

hipError_t launch_grouped_gate_up(const _Float16 *x16, int K, const ExpertWeights &ew, int F, const BucketOut &b,
                                  _Float16 *h16, hipStream_t s)
{
    // any split of the n tiles into runs (the bucketing wrote rpi_gu runs per work item)
    if (ew.gate_type != ew.up_type || ew.gate_stride != ew.up_stride || !grouped_type_ok(ew.gate_type, K) ||
        b.tile_m != GG_TILE_M || !grouped_shape_ok(K, F) || b.runs_gu == nullptr || b.desc_gu == nullptr ||
        b.rpi_gu < 1 || b.rpi_gu > F / GG_TILE_N || b.max_tiles < 1)
        return hipErrorInvalidValue;
    switch (ew.gate_type) {
    case T_Q4_K: return gate_up_t<T_Q4_K>(x16, K, ew, F, b, h16, s);
    case T_Q6_K: return gate_up_t<T_Q6_K>(x16, K, ew, F, b, h16, s);
    case T_Q8_0: return gate_up_t<T_Q8_0>(x16, K, ew, F, b, h16, s);
    default: return hipErrorInvalidValue;
    }
}

template <int TV>
static hipError_t dense_t(const _Float16 *x16, int K, const ExpertWeights &ew, int N, const BucketOut &b, float *c,
                          hipStream_t s)
{
    // one n tile per run: a dense product has few token tiles, so the runs,
    // not the tiles, must fill the CUs
    const unsigned grid = gg_grid(b.max_tiles * b.rpi_gu);
    hipLaunchKernelGGL((k_grouped_gate_up<TV, true>), dim3(grid), dim3(64 * GG_WV), 0, s, x16, K, ew, N / 2, b,
                       nullptr, 1, c);
    return hipGetLastError();
}

bool dense_mfma_shape_ok(int type, int N, int K)
{
    return grouped_type_ok(type, K) && K % (256 * DS3_GU_DEPTH) == 0 && N > 0 && N % (2 * GG_TILE_N) == 0;
}

int dense_runs_per_tile(int N) { return N / 2 / GG_TILE_N; }

hipError_t launch_dense_mfma(const _Float16 *x16, int K, const uint8_t *w, uint64_t stride, int type, int N,
                             const BucketOut &b, float *c, hipStream_t s)
{
    const int rg = dense_runs_per_tile(N);
    const uint64_t row_b = type == T_Q8_0 ? (uint64_t)(K / 32) * 34 : (uint64_t)(K / 256) * (type == T_Q4_K ? 144 : 210);
    if (!dense_mfma_shape_ok(type, N, K) || b.tile_m != GG_TILE_M || b.runs_gu == nullptr || b.desc_gu == nullptr ||
        b.rpi_gu != rg || b.max_tiles < 1 ||
        stride < row_b)
        return hipErrorInvalidValue;
    ExpertWeights ew{};
    ew.gate = w;
    ew.up = w + (uint64_t)(N / 2) * stride;
    ew.down = nullptr;
    ew.gate_stride = ew.up_stride = stride;
    ew.gate_type = ew.up_type = type;
    ew.table = nullptr;
    switch (type) {
    case T_Q4_K: return dense_t<T_Q4_K>(x16, K, ew, N, b, c, s);
    case T_Q6_K: return dense_t<T_Q6_K>(x16, K, ew, N, b, c, s);
    case T_Q8_0: return dense_t<T_Q8_0>(x16, K, ew, N, b, c, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_grouped_down(const _Float16 *h16, int F, const ExpertWeights &ew, int N, const BucketOut &b,
                               _Float16 *y, hipStream_t s)
{
    const int rd = (N / GG_TILE_N + DS3_DN_NTB - 1) / DS3_DN_NTB;
    if (!grouped_type_ok(ew.down_type, F) || b.tile_m != GG_TILE_M || !grouped_shape_ok(N, F) ||
        b.runs_dn == nullptr || b.desc_dn == nullptr || b.rpi_dn != rd || b.max_tiles < 1)
        return hipErrorInvalidValue;
    switch (ew.down_type) {
    case T_Q4_K: return down_t<T_Q4_K>(h16, F, ew, N, b, y, s);
    case T_Q6_K: return down_t<T_Q6_K>(h16, F, ew, N, b, y, s);
    case T_Q8_0: return down_t<T_Q8_0>(h16, F, ew, N, b, y, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ds3k
