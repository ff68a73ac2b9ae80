// moe_prefill.hip -- grouped expert products for many tokens (prefill).
//
// Replaces the reference's per-expert gather -> matmul_quantized_batch x3 ->
// silu_mul -> scatter sequence (src/ds3_engine.c:969-1016,
// metal/matmul_q4k.metal:247-286) with two MFMA kernels over the bucketed
// token lists:
//   gate_up: H[pos][r] = silu(X_e . Wg_e[r]) * (X_e . Wu_e[r])   (fp16 out)
//   down:    Y[pos][j] = H_e[pos] . Wd_e[j]                       (fp32 out)
// where pos runs over expert e's compacted token positions.
//
// Precision: operands are fp16 (x, dequantised weights, h), accumulation is
// fp32 in v_mfma_f32_16x16x32_f16.  Each weight is one fp32-precision FMA on
// its code rounded once to fp16.
//
// Work decomposition.  A work item is (expert, 64-token tile) from the
// bucketing kernel; a run is one item and a few consecutive 128-row output
// tiles, walked as one flat sequence of 256-wide K steps.  Workgroups are
// persistent (one per CU) and take runs in an XCD-aware order.  Each of the 8
// waves owns 16 output rows (one MFMA column block; for gate_up the same rows
// of gate and up, so SwiGLU happens in registers).
//
// Weight stream.  Every wave streams its own rows' quantised bytes straight
// into a private LDS ring of D stages with global_load_lds_dwordx4 (no
// registers are spent on staging, so D-1 steps of weights stay in flight),
// waits for the stage with s_waitcnt vmcnt, copies its units from LDS into
// registers (common.h RawUnits) and decodes them to fp16 MFMA fragments.  The
// 64-token activation tile of each step is staged through registers into LDS
// and shared by the 8 waves.  Per 256-wide K step, lane group g (lanes
// 16g..16g+15) holds units g and g+4 of its row (see common.h); K-slot q of
// the step is segment q%4 of unit g+4*(q/4), and the A fragment is read from
// the same K positions, so the MFMA's K order is a permutation shared by both
// operands.
#include "common.h"
#include "launch.h"

namespace ds3k {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // a native vector: copies stay in registers

constexpr int GM_TILE_M = 64;
// Activation tile rows in LDS: 512 bytes (256 halves) each, 16-byte chunk c
// of row r at r * 512 + 16 * (c ^ (r & 15)).  The XOR swizzle spreads the 16
// rows one fragment read touches over the banks with no padding, so one
// 64-lane DMA fills two whole rows.
constexpr int GM_ROWB = 512;
constexpr int N_XCD = 8;                  // MI355X: workgroups go round-robin to 8 XCDs

#define DS3_LDS __attribute__((address_space(3)))

__device__ __forceinline__ const uint8_t *ebase(const uint8_t *base, const uint64_t *table, int e, int which,
                                                uint64_t rows, uint64_t stride)
{
    return base + (table ? table[3 * e + which] : (uint64_t)e * rows * stride);
}

// Weight ring geometry.  BLK = quantised bytes of one row per 256-wide K
// step; a stage holds CPR 16-byte chunks per row.  Q4_K rows are 16-byte
// aligned in GGUF files, so a step's block is exactly 9 chunks;
// Q6_K / Q8_0 blocks start anywhere, so the chunk run starts at the aligned
// address below the block and covers 15 bytes of slack.  (An expert whose
// Q4_K rows are not 16-byte aligned is read in place instead.)
template <int TYPE> struct WGeo;
template <> struct WGeo<T_Q4_K> { static constexpr int BLK = 144, CPR = 9; static constexpr bool ALIGNED = true; };
template <> struct WGeo<T_Q6_K> { static constexpr int BLK = 210, CPR = 15; static constexpr bool ALIGNED = false; };
template <> struct WGeo<T_Q8_0> { static constexpr int BLK = 272, CPR = 18; static constexpr bool ALIGNED = false; };

// A weight stage is padded to whole DMA instructions (64 chunks) so that
// every lane issues every instruction: lanes past the last chunk repeat
// chunk 0 into the padding.
// LDS layout of one workgroup (bytes): two activation tiles (64 rows of
// GM_ROWB bytes) then two weight stages per wave.  WV = waves per workgroup
// (16 output rows each): 8 where that fits 160 KiB of LDS, else 4.
constexpr int GM_ATILE = GM_TILE_M * GM_ROWB;
constexpr int GM_LDS_MAX = 163840;
template <int TYPE, int NB> struct GmCfg {
    static constexpr int CPR = WGeo<TYPE>::CPR;
    static constexpr int NI = (NB * 16 * CPR + 63) / 64;       // DMA instructions per stage
    static constexpr int STAGE = NI * 1024;                    // bytes per wave per stage
    static constexpr int WV = 2 * GM_ATILE + 2 * 8 * STAGE <= GM_LDS_MAX ? 8 : 4;
    static constexpr int TILE_N = 16 * WV;
    static constexpr int LDS = 2 * GM_ATILE + 2 * WV * STAGE;
    static_assert(LDS <= GM_LDS_MAX, "workgroup LDS exceeds the CU's 160 KiB");
};

// Workgroup barrier for LDS traffic: waits for this wave's LDS operations,
// then s_barrier.  Vector memory is waited for separately.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ void vm_wait_all()
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// 16-byte global -> LDS DMA: lane i writes lds + 16*i.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds)
{
    __builtin_amdgcn_global_load_lds(src, (DS3_LDS void *)(uintptr_t)lds, 16, 0, 0);
}

// A fragment reads for K slots 4*hv + 2*pp + {0, 1}: MB row blocks each,
// all issued before one wait; the wait names every result so nothing reads
// them early.  Lane (g, m) reads row 16*mb + m: rowbase (row m) + the
// swizzled chunk + 16 * GM_ROWB * mb.
template <int TYPE, int MB>
__device__ __forceinline__ void a_frags(uint32_t rowbase, int g, int m, int hv, int pp, half8 (&af)[2][4])
{
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const uint32_t c = (uint32_t)slot_k0<TYPE>(0, g, 4 * hv + 2 * pp + p) / 8u;
        const uint32_t a = rowbase + 16u * (c ^ (uint32_t)m);
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(af[p][mb]) : "v"(a), "i"(16 * GM_ROWB * mb));
    }
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

// One 256-wide K step for NB column blocks of 16 rows (gate/up: NB = 2,
// gate and up of the same rows; down: NB = 1), weights from `raw`, the
// activation tile at LDS byte address `as`.
template <int TYPE, int NB, int MB>
__device__ __forceinline__ void gm_step(uint32_t as, const RawUnits<TYPE> (&raw)[NB], int lane,
                                        floatx4 (&acc)[4][NB])
{
    const int g = lane >> 4, m = lane & 15;
    const uint32_t rowbase = as + (uint32_t)(m * GM_ROWB);
#pragma unroll
    for (int hv = 0; hv < 2; hv++) {
        half8 bq[NB][4];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) raw[nb].decode_frags(hv, g, bq[nb]);
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            half8 af[2][4];
            a_frags<TYPE, MB>(rowbase, g, m, hv, pp, af);
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[p][mb], bq[nb][2 * pp + p], acc[mb][nb],
                                                                              0, 0, 0);
        }
    }
}

constexpr int GM_MAX_NI = 12;      // weight DMA instructions per stage the run state can hold

// A run: one work item and nnt consecutive 128-row n tiles, walked as a flat
// sequence of U = nnt * S K steps (step u: n tile nt0 + u / S, K step u % S),
// so the streams stay in flight across n-tile boundaries.
template <int NB>
struct GmRun {
    const _Float16 *a_src;
    uint32_t a_row[8];              // DMA j: element offset of this lane's source chunk (row pair wave + WV*j)
    const uint8_t *rows[NB];        // this lane's weight row in n tile nt0 (decode side)
    const uint8_t *wave_rows[NB];   // the wave's first weight row in n tile nt0, per column block
    uint32_t dma_off[GM_MAX_NI];    // this lane's chunk of DMA instruction i: row * stride of its row
                                    // (bits 0..23) and its 16-byte part in the row's run (bits 24..31)
    uint32_t dma_nb;                // bit i: column block of that chunk
    uint64_t tstride;               // bytes between the same row of consecutive n tiles
    int S, nt0, U, lane, wave;
    uint32_t lds;                   // LDS byte address of the workgroup's area
    bool w_dma;                     // weights stream through the LDS ring (else: read in place)
};

// Loads of flat step v into buffer v & 1, all by DMA: the activation row
// pairs wave + WV*j below 8*MB (rows past the tile's tokens repeat its first
// row; 64 lanes x 16 bytes fill two swizzled rows) and this wave's weight
// stage.
template <int TYPE, int NB, int MB>
__device__ __forceinline__ void gm_issue(const GmRun<NB> &r, int v)
{
    using C = GmCfg<TYPE, NB>;
    static_assert(8 * MB % C::WV == 0 && 8 * MB / C::WV <= 8 && C::NI <= GM_MAX_NI, "run state arrays too small");
    using G = WGeo<TYPE>;
    const int buf = v & 1;
    const int wt = v / r.S, ws = v - wt * r.S;
    {
        const uint32_t at = r.lds + (uint32_t)(buf * GM_ATILE);
#pragma unroll
        for (int j = 0; j < 8 * MB / C::WV; j++)
            dma16(r.a_src + r.a_row[j] + 256 * ws, at + (uint32_t)(2 * GM_ROWB * (r.wave + C::WV * j)));
    }
    if (!r.w_dma) return;
    const uint64_t step_off = (uint64_t)wt * r.tstride + (uint64_t)ws * G::BLK;
    const uint32_t dst = r.lds + (uint32_t)(2 * GM_ATILE + (buf * C::WV + r.wave) * C::STAGE);
#pragma unroll
    for (int i = 0; i < C::NI; i++) {
        const uint8_t *wr = r.wave_rows[0];
        if constexpr (NB > 1) wr = ((r.dma_nb >> i) & 1u) ? r.wave_rows[1] : r.wave_rows[0];
        uintptr_t blk = (uintptr_t)(wr + (r.dma_off[i] & 0xffffffu) + step_off);
        if constexpr (!G::ALIGNED) blk &= ~(uintptr_t)15;
        dma16((const void *)(blk + 16u * (r.dma_off[i] >> 24)), dst + 1024u * (uint32_t)i);
    }
}

// Per step u: wait for this wave's DMAs of step u (issued one step ahead),
// barrier (every wave's share of the activation tile has landed, and every
// wave is done with buffer (u+1) & 1), issue the loads of step u+1, compute
// step u.  vmcnt(0) holds whatever order the memory system returns in.
// (A third weight stage for tiles of at most 32 tokens, and stores deferred
// by one step, measured no faster on MI355X at T = 512.)
template <int TYPE, int NB, int MB, bool INPLACE, class Epi>
__device__ __forceinline__ void gm_run(const GmRun<NB> &r, const Epi &epi)
{
    using C = GmCfg<TYPE, NB>;
    using G = WGeo<TYPE>;
    const int last = r.U - 1, q = r.lane >> 4, m = r.lane & 15;
    floatx4 acc[4][NB];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };
    gm_issue<TYPE, NB, MB>(r, 0);
    for (int u = 0; u < r.U; u++) {
        const int ct = u / r.S, cs = u - ct * r.S, buf = u & 1;
        vm_wait_all();
        lds_barrier();
        if (u < last) gm_issue<TYPE, NB, MB>(r, u + 1);
        RawUnits<TYPE> cur[NB];
        const uint32_t stage = r.lds + (uint32_t)(2 * GM_ATILE + (buf * C::WV + r.wave) * C::STAGE);
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const uint32_t row_at = stage + (uint32_t)((nb * 16 + m) * C::CPR * 16);
            if constexpr (G::ALIGNED) {
                // Q4_K rows are 16-byte aligned in every GGUF file; an expert
                // whose rows are not is read in place, slowly but exactly
                if constexpr (!INPLACE) cur[nb].load_lds(row_at, q);
                else cur[nb].load_global(r.rows[nb] + (uint64_t)ct * r.tstride + (uint64_t)cs * G::BLK, q);
            } else {
                const int sh = (int)((uintptr_t)(r.rows[nb] + (uint64_t)ct * r.tstride + (uint64_t)cs * G::BLK) & 15);
                cur[nb].load_lds(row_at, sh, q);
            }
        }
        gm_step<TYPE, NB, MB>(r.lds + (uint32_t)(buf * GM_ATILE), cur, r.lane, acc);
        if (cs == r.S - 1) {
            typename Epi::template Out<MB> o;
            epi.template finish<MB>(acc, r.nt0 + ct, o);
            epi.template store<MB>(o);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < NB; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };
        }
    }
    lds_barrier();                  // everyone is done with the buffers before the next run
}

template <int TYPE, int NB, bool INPLACE, class Epi>
__device__ __forceinline__ void gm_run_mb(int mblocks, const GmRun<NB> &r, const Epi &epi)
{
    switch (mblocks) {
    case 1: gm_run<TYPE, NB, 1, INPLACE>(r, epi); break;
    case 2: gm_run<TYPE, NB, 2, INPLACE>(r, epi); break;
    case 3: gm_run<TYPE, NB, 3, INPLACE>(r, epi); break;
    default: gm_run<TYPE, NB, 4, INPLACE>(r, epi); break;
    }
}

// Runs whose Q4_K rows are not 16-byte aligned (never in GGUF files) read
// their weights in place, through a separate instantiation so the hot path
// keeps its registers.
template <int TYPE, int NB, class Epi>
__device__ __forceinline__ void gm_run_any(int mblocks, const GmRun<NB> &r, const Epi &epi)
{
    if constexpr (WGeo<TYPE>::ALIGNED) {
        if (!r.w_dma) {
            gm_run_mb<TYPE, NB, true>(mblocks, r, epi);
            return;
        }
    }
    gm_run_mb<TYPE, NB, false>(mblocks, r, epi);
}

// Work item header shared by both kernels.
struct GmItem {
    int e, off, m0, mrows, mblocks;
};
__device__ __forceinline__ bool gm_item(const BucketOut &b, int item, GmItem &it)
{
    if (item >= *b.n_tiles) return false;
    const int packed = b.tiles[item];
    it.e = packed >> 16;
    const int mt = packed & 0xffff;
    it.off = b.offsets[it.e];
    it.m0 = mt * GM_TILE_M;
    it.mrows = min(GM_TILE_M, b.counts[it.e] - it.m0);
    it.mblocks = (it.mrows + 15) / 16;
    return true;
}

// Persistent schedule: run index r = blockIdx.x + k * gridDim.x (gridDim.x a
// multiple of 8, so r % 8 is the workgroup's XCD) maps to (item, run) with
// every run of one item on the same XCD, whose L2 then holds that item's
// activation rows.
__device__ __forceinline__ void gm_decode_run(int r, int runs_per_item, int &item, int &run)
{
    const int local = r / N_XCD;
    item = N_XCD * (local / runs_per_item) + r % N_XCD;
    run = local % runs_per_item;
}

// Lane-constant part of a run: the DMA chunk map of this lane.  Chunk
// c = 64*i + lane of a stage is (column block c / (16*CPR), row
// (c / CPR) % 16, part c % CPR); lanes past the last chunk repeat chunk 0.
template <int TYPE, int NB>
__device__ __forceinline__ void gm_dma_map(GmRun<NB> &r, int lane, uint64_t stride)
{
    using C = GmCfg<TYPE, NB>;
    static_assert(C::NI <= GM_MAX_NI && C::CPR < 256, "more weight DMA instructions per stage than GmRun holds");
    r.dma_nb = 0u;
#pragma unroll
    for (int i = 0; i < C::NI; i++) {
        const int c0 = 64 * i + lane, c = c0 < NB * 16 * C::CPR ? c0 : 0;
        const int nb = c / (16 * C::CPR), row = (c / C::CPR) % 16;
        r.dma_off[i] = (uint32_t)(row * stride) | ((uint32_t)(c % C::CPR) << 24);
        r.dma_nb |= (uint32_t)nb << i;
    }
}

// Epilogues: finish() turns a tile's accumulators into output values held
// in registers (Out), store() writes them.  Lane (g = lane/16, m = lane%16)
// of wave w holds rows 16mb + 4g + j of output column nt*tile_n + 16w + m.
struct EpiGateUp {
    _Float16 *h16;
    int F, row0, mrows, tile_n;       // row0 = compacted position of the tile's first token
    template <int MB> struct Out {
        _Float16 v[MB][4];
        int nt;
    };
    template <int MB>
    __device__ __forceinline__ void finish(const floatx4 (&acc)[4][2], int nt, Out<MB> &o) const
    {
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int j = 0; j < 4; j++) o.v[mb][j] = (_Float16)swiglu(acc[mb][0][j], acc[mb][1][j]);
        o.nt = nt;
    }
    template <int MB>
    __device__ __forceinline__ void store(const Out<MB> &o) const
    {
        const int lane = threadIdx.x & 63;
        const int nrow = o.nt * tile_n + 16 * (threadIdx.x >> 6) + (lane & 15);
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int mr = 16 * mb + 4 * (lane >> 4) + j;
                if (mr < mrows) h16[(int64_t)(row0 + mr) * F + nrow] = o.v[mb][j];
            }
        }
    }
};

struct EpiDown {
    float *y;
    int N, row0, mrows, tile_n;
    template <int MB> struct Out {
        float v[MB][4];
        int nt;
    };
    template <int MB>
    __device__ __forceinline__ void finish(const floatx4 (&acc)[4][1], int nt, Out<MB> &o) const
    {
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int j = 0; j < 4; j++) o.v[mb][j] = acc[mb][0][j];
        o.nt = nt;
    }
    template <int MB>
    __device__ __forceinline__ void store(const Out<MB> &o) const
    {
        const int lane = threadIdx.x & 63;
        const int nrow = o.nt * tile_n + 16 * (threadIdx.x >> 6) + (lane & 15);
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int mr = 16 * mb + 4 * (lane >> 4) + j;
                if (mr < mrows) y[(int64_t)(row0 + mr) * N + nrow] = o.v[mb][j];
            }
        }
    }
};

template <int TYPE>
__global__ void __launch_bounds__((64 * GmCfg<TYPE, 2>::WV))
k_grouped_gate_up(const _Float16 *__restrict__ x16, int K, ExpertWeights ew, int F, BucketOut b,
                  _Float16 *__restrict__ h16, int ntb, int n_runs)
{
    using C = GmCfg<TYPE, 2>;
    __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS];
    const int n_nt = F / C::TILE_N, runs_per_item = (n_nt + ntb - 1) / ntb;
    // the wave index as a uniform value keeps wave-derived pointers in SGPRs
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int rr = blockIdx.x; rr < n_runs; rr += gridDim.x) {
        int item, run;
        gm_decode_run(rr, runs_per_item, item, run);
        GmItem it;
        if (!gm_item(b, item, it)) continue;            // uniform over the workgroup
        GmRun<2> r;
        r.lane = lane;
        r.wave = wave;
        r.a_src = x16;
#pragma unroll
        for (int j = 0; j < 32 / C::WV; j++) {
            const int row = 2 * (wave + C::WV * j) + (lane >> 5), chunk = (lane & 31) ^ (row & 15);
            r.a_row[j] = (uint32_t)b.ids[it.off + it.m0 + (row < it.mrows ? row : 0)] * (uint32_t)K + 8u * chunk;
        }
        r.nt0 = run * ntb;
        const int nnt = min(ntb, n_nt - r.nt0);
        const uint8_t *wg = ebase(ew.gate, ew.table, it.e, 0, (uint64_t)F, ew.gate_stride);
        const uint8_t *wu = ebase(ew.up, ew.table, it.e, 1, (uint64_t)F, ew.up_stride);
        const size_t wrow0 = (size_t)r.nt0 * C::TILE_N + 16 * wave;
        const uint8_t *wave_rows[2] = { wg + wrow0 * ew.gate_stride, wu + wrow0 * ew.up_stride };
        r.rows[0] = wave_rows[0] + (size_t)(lane & 15) * ew.gate_stride;
        r.rows[1] = wave_rows[1] + (size_t)(lane & 15) * ew.up_stride;
        r.wave_rows[0] = wave_rows[0];
        r.wave_rows[1] = wave_rows[1];
        gm_dma_map<TYPE, 2>(r, lane, ew.gate_stride);      // gate and up strides are equal
        r.tstride = (uint64_t)C::TILE_N * ew.gate_stride;
        r.w_dma = !WGeo<TYPE>::ALIGNED || ((((uintptr_t)wg | (uintptr_t)wu | ew.gate_stride) & 15) == 0);
        r.S = K / 256;
        r.U = nnt * r.S;
        r.lds = (uint32_t)(uintptr_t)(DS3_LDS void *)smem;
        const EpiGateUp epi{ h16, F, it.off + it.m0, it.mrows, C::TILE_N };
        gm_run_any<TYPE, 2>(it.mblocks, r, epi);
    }
}

template <int TYPE>
__global__ void __launch_bounds__((64 * GmCfg<TYPE, 1>::WV))
k_grouped_down(const _Float16 *__restrict__ h16, int F, ExpertWeights ew, int N, BucketOut b,
               float *__restrict__ y, int ntb, int n_runs)
{
    using C = GmCfg<TYPE, 1>;
    __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS];
    const int n_nt = N / C::TILE_N, runs_per_item = (n_nt + ntb - 1) / ntb;
    // the wave index as a uniform value keeps wave-derived pointers in SGPRs
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int rr = blockIdx.x; rr < n_runs; rr += gridDim.x) {
        int item, run;
        gm_decode_run(rr, runs_per_item, item, run);
        GmItem it;
        if (!gm_item(b, item, it)) continue;            // uniform over the workgroup
        GmRun<1> r;
        r.lane = lane;
        r.wave = wave;
        r.a_src = h16;
#pragma unroll
        for (int j = 0; j < 32 / C::WV; j++) {
            const int row = 2 * (wave + C::WV * j) + (lane >> 5), chunk = (lane & 31) ^ (row & 15);
            r.a_row[j] = (uint32_t)(it.off + it.m0 + (row < it.mrows ? row : 0)) * (uint32_t)F + 8u * chunk;
        }
        r.nt0 = run * ntb;
        const int nnt = min(ntb, n_nt - r.nt0);
        const uint8_t *wd = ebase(ew.down, ew.table, it.e, 2, (uint64_t)N, ew.down_stride);
        const uint8_t *wave_rows[1] = { wd + ((size_t)r.nt0 * C::TILE_N + 16 * wave) * ew.down_stride };
        r.rows[0] = wave_rows[0] + (size_t)(lane & 15) * ew.down_stride;
        r.wave_rows[0] = wave_rows[0];
        gm_dma_map<TYPE, 1>(r, lane, ew.down_stride);
        r.tstride = (uint64_t)C::TILE_N * ew.down_stride;
        r.w_dma = !WGeo<TYPE>::ALIGNED || ((((uintptr_t)wd | ew.down_stride) & 15) == 0);
        r.S = F / 256;
        r.U = nnt * r.S;
        r.lds = (uint32_t)(uintptr_t)(DS3_LDS void *)smem;
        const EpiDown epi{ y, N, it.off + it.m0, it.mrows, C::TILE_N };
        gm_run_any<TYPE, 1>(it.mblocks, r, epi);
    }
}

bool grouped_type_ok(int type, int K)
{
    if (K <= 0 || K % 256 != 0) return false;
    return type == T_Q4_K || type == T_Q6_K || type == T_Q8_0;
}

// n tiles per run (tuning knobs): at T = 512 (about 128 work items) these
// give each persistent workgroup one long run (gate_up: 2 runs of 3 n tiles
// per item; down: 2 runs of 8), so the stream's start-up latency is paid
// once per workgroup.
#ifndef DS3_GU_NTB
#define DS3_GU_NTB 3
#endif
#ifndef DS3_DN_NTB
#define DS3_DN_NTB 8
#endif

// Persistent grid: one workgroup per CU (a multiple of 8), walking
// n_runs = 8 * ceil(max_items / 8) * runs_per_item runs.
static void gm_grid(int n_nt, int ntb, int max_items, unsigned &grid, int &n_runs)
{
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    const int runs_per_item = (n_nt + ntb - 1) / ntb;
    n_runs = N_XCD * ((max_items + N_XCD - 1) / N_XCD) * runs_per_item;
    const int g = (n_cu + N_XCD - 1) / N_XCD * N_XCD;
    grid = (unsigned)(n_runs < g ? n_runs : g);
}

template <int TV>
static hipError_t gate_up_t(const _Float16 *x16, int K, const ExpertWeights &ew, int F, const BucketOut &b,
                            _Float16 *h16, hipStream_t s)
{
    using C = GmCfg<TV, 2>;
    if (F % C::TILE_N != 0) return hipErrorInvalidValue;
    unsigned grid;
    int n_runs;
    gm_grid(F / C::TILE_N, DS3_GU_NTB, b.max_tiles, grid, n_runs);
    hipLaunchKernelGGL((k_grouped_gate_up<TV>), dim3(grid), dim3(64 * C::WV), 0, s, x16, K, ew, F, b, h16, DS3_GU_NTB,
                       n_runs);
    return hipGetLastError();
}

template <int TV>
static hipError_t down_t(const _Float16 *h16, int F, const ExpertWeights &ew, int N, const BucketOut &b, float *y,
                         hipStream_t s)
{
    using C = GmCfg<TV, 1>;
    if (N % C::TILE_N != 0) return hipErrorInvalidValue;
    unsigned grid;
    int n_runs;
    gm_grid(N / C::TILE_N, DS3_DN_NTB, b.max_tiles, grid, n_runs);
    hipLaunchKernelGGL((k_grouped_down<TV>), dim3(grid), dim3(64 * C::WV), 0, s, h16, F, ew, N, b, y, DS3_DN_NTB,
                       n_runs);
    return hipGetLastError();
}

hipError_t launch_grouped_gate_up(const _Float16 *x16, int K, const ExpertWeights &ew, int F, const BucketOut &b,
                                  _Float16 *h16, hipStream_t s)
{
    if (ew.gate_type != ew.up_type || ew.gate_stride != ew.up_stride || !grouped_type_ok(ew.gate_type, K) ||
        b.tile_m != GM_TILE_M)
        return hipErrorInvalidValue;
    switch (ew.gate_type) {
    case T_Q4_K: return gate_up_t<T_Q4_K>(x16, K, ew, F, b, h16, s);
    case T_Q6_K: return gate_up_t<T_Q6_K>(x16, K, ew, F, b, h16, s);
    case T_Q8_0: return gate_up_t<T_Q8_0>(x16, K, ew, F, b, h16, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_grouped_down(const _Float16 *h16, int F, const ExpertWeights &ew, int N, const BucketOut &b,
                               float *y, hipStream_t s)
{
    if (!grouped_type_ok(ew.down_type, F) || b.tile_m != GM_TILE_M) return hipErrorInvalidValue;
    switch (ew.down_type) {
    case T_Q4_K: return down_t<T_Q4_K>(h16, F, ew, N, b, y, s);
    case T_Q6_K: return down_t<T_Q6_K>(h16, F, ew, N, b, y, s);
    case T_Q8_0: return down_t<T_Q8_0>(h16, F, ew, N, b, y, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ds3k
