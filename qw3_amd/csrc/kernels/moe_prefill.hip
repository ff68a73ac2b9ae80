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
// Work decomposition: blockIdx.y = work item (expert, 64-token tile) from the
// bucketing kernel, blockIdx.x = 128-row output tile.  Each of the 8 waves
// owns 16 output rows (one MFMA column block; for gate_up the same rows of
// gate and up, so SwiGLU happens in registers), decodes their weight
// fragments in registers (common.h RawUnits::decode_frags) and applies them
// to all 16-token row blocks of the tile, which sit in LDS as fp16.  Weight
// bytes of step s+1 load while step s computes.  Per 256-wide
// K step, lane group g (lanes 16g..16g+15) holds units g and g+4 of its row
// (see common.h); K-slot q of the step is segment q%4 of unit g+4*(q/4), and
// the A fragment is read from the same K positions, so the MFMA's K order is a
// permutation shared by both operands.
#include "common.h"
#include "launch.h"

namespace ds3k {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int GM_TILE_M = 64;
constexpr int GM_WAVES = 8;
constexpr int GM_TPB = GM_WAVES * 64;
constexpr int GM_ROW = 256 + 8;           // halves per LDS row (16-byte pad)
constexpr int GM_TILE_N = 16 * GM_WAVES;  // output rows per workgroup (16 per wave)
constexpr int GM_ACH = GM_TILE_M * 32 / GM_TPB;   // 16-byte A chunks per thread per K step

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

__device__ __forceinline__ const uint8_t *ebase(const uint8_t *base, const uint64_t *table, int e, int which,
                                                uint64_t rows, uint64_t stride)
{
    return base + (table ? table[3 * e + which] : (uint64_t)e * rows * stride);
}

// A tile of one K step: 64 rows x 32 chunks of 16 bytes (rows beyond the
// tile are zero); thread covers rows (tid>>5) + (GM_TPB/32)*i, chunk tid&31.
struct ATile {
    uint4 r[GM_ACH];
};

__device__ __forceinline__ void a_load(ATile &a, const _Float16 *src, const int64_t (&row_off)[GM_ACH], int s,
                                       int chunk)
{
#pragma unroll
    for (int i = 0; i < GM_ACH; i++) {
        if (row_off[i] >= 0) a.r[i] = *(const uint4 *)(src + row_off[i] + 256 * s + 8 * chunk);
        else a.r[i] = make_uint4(0u, 0u, 0u, 0u);
    }
}

__device__ __forceinline__ void a_store(const ATile &a, _Float16 *As, int row0, int chunk)
{
#pragma unroll
    for (int i = 0; i < GM_ACH; i++) *(uint4 *)(As + (row0 + (GM_TPB / 32) * i) * GM_ROW + 8 * chunk) = a.r[i];
}

// One 256-wide K step for NB column blocks of 16 rows (gate/up: NB = 2,
// gate and up of the same rows; down: NB = 1), weights from `raw`.
template <int TYPE, int NB, int MB>
__device__ __forceinline__ void gm_step(const _Float16 *As, const RawUnits<TYPE> (&raw)[NB], int s, int lane,
                                        floatx4 (&acc)[4][NB])
{
    const int g = lane >> 4, m = lane & 15;
#pragma unroll
    for (int hv = 0; hv < 2; hv++) {
        half8 bq[NB][4];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) raw[nb].decode_frags(hv, g, bq[nb]);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int col = slot_k0<TYPE>(s, g, 4 * hv + p) - 256 * s;
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
                const half8 a = *(const half8 *)(As + (16 * mb + m) * GM_ROW + col);
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[nb][p], acc[mb][nb], 0, 0, 0);
            }
        }
    }
}

// One step of the K loop: publish the A tile of step s, start the loads of
// step s+1 (A into registers, weights into `nxt`), then compute step s.
template <int TYPE, int NB, int MB>
__device__ __forceinline__ void gm_iter(const _Float16 *a_src, const int64_t (&row_off)[GM_ACH], int arow0,
                                        int achunk, const uint8_t *const (&rows)[NB], int s, int S, int lane,
                                        _Float16 *As, ATile &a, const RawUnits<TYPE> (&cur)[NB],
                                        RawUnits<TYPE> (&nxt)[NB], floatx4 (&acc)[4][NB])
{
    __syncthreads();
    a_store(a, As, arow0, achunk);
    __syncthreads();
    if (s + 1 < S) {
        a_load(a, a_src, row_off, s + 1, achunk);
#pragma unroll
        for (int nb = 0; nb < NB; nb++) nxt[nb].load(rows[nb], s + 1, lane >> 4);
    }
    gm_step<TYPE, NB, MB>(As, cur, s, lane, acc);
}

// K loop shared by both kernels; two raw buffers alternate so staged weight
// bytes are never copied.
// MB = number of 16-token row blocks with data (1..4), a template parameter
// so the MFMA sequence has no data-dependent branches.
template <int TYPE, int NB, int MB>
__device__ __forceinline__ void gm_kloop(const _Float16 *a_src, const int64_t (&row_off)[GM_ACH], int arow0, int achunk,
                                         const uint8_t *const (&rows)[NB], int S, int lane,
                                         _Float16 *As, floatx4 (&acc)[4][NB])
{
    ATile a;
    a_load(a, a_src, row_off, 0, achunk);
    RawUnits<TYPE> r0[NB], r1[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) r0[nb].load(rows[nb], 0, lane >> 4);
    for (int s = 0; s < S; s += 2) {
        gm_iter<TYPE, NB, MB>(a_src, row_off, arow0, achunk, rows, s, S, lane, As, a, r0, r1, acc);
        if (s + 1 < S)
            gm_iter<TYPE, NB, MB>(a_src, row_off, arow0, achunk, rows, s + 1, S, lane, As, a, r1, r0, acc);
    }
}

template <int TYPE, int NB>
__device__ __forceinline__ void gm_kloop_mb(int mblocks, const _Float16 *a_src, const int64_t (&row_off)[GM_ACH],
                                            int arow0, int achunk, const uint8_t *const (&rows)[NB], int S, int lane,
                                            _Float16 *As, floatx4 (&acc)[4][NB])
{
    switch (mblocks) {
    case 1: gm_kloop<TYPE, NB, 1>(a_src, row_off, arow0, achunk, rows, S, lane, As, acc); break;
    case 2: gm_kloop<TYPE, NB, 2>(a_src, row_off, arow0, achunk, rows, S, lane, As, acc); break;
    case 3: gm_kloop<TYPE, NB, 3>(a_src, row_off, arow0, achunk, rows, S, lane, As, acc); break;
    default: gm_kloop<TYPE, NB, 4>(a_src, row_off, arow0, achunk, rows, S, lane, As, acc); break;
    }
}

template <int TYPE>
__global__ void __launch_bounds__(GM_TPB)
k_grouped_gate_up(const _Float16 *__restrict__ x16, int K, ExpertWeights ew, int F, BucketOut b,
                  _Float16 *__restrict__ h16)
{
    __shared__ __attribute__((aligned(16))) _Float16 As[GM_TILE_M * GM_ROW];
    const int item = blockIdx.y;
    if (item >= *b.n_tiles) return;
    const int packed = b.tiles[item];
    const int e = packed >> 16, mt = packed & 0xffff;
    const int off = b.offsets[e], c_e = b.counts[e];
    const int m0 = mt * GM_TILE_M;
    const int mrows = min(GM_TILE_M, c_e - m0);
    const int mblocks = (mrows + 15) / 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    const int arow0 = tid >> 5, achunk = tid & 31;
    int64_t row_off[GM_ACH];
#pragma unroll
    for (int i = 0; i < GM_ACH; i++) {
        const int r = arow0 + (GM_TPB / 32) * i;
        row_off[i] = r < mrows ? (int64_t)b.ids[off + m0 + r] * K : -1;
    }

    const uint8_t *wg = ebase(ew.gate, ew.table, e, 0, (uint64_t)F, ew.gate_stride);
    const uint8_t *wu = ebase(ew.up, ew.table, e, 1, (uint64_t)F, ew.up_stride);
    const int nrow = blockIdx.x * GM_TILE_N + 16 * wave + (lane & 15);
    const uint8_t *rows[2] = { wg + (size_t)nrow * ew.gate_stride, wu + (size_t)nrow * ew.up_stride };

    floatx4 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };

    gm_kloop_mb<TYPE, 2>(mblocks, x16, row_off, arow0, achunk, rows, K / 256, lane, As, acc);

    // Epilogue: lane holds rows 4*(lane>>4)+j of each 16-row block, column lane&15.
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int mr = 16 * mb + 4 * (lane >> 4) + j;
            if (mr < mrows)
                h16[(int64_t)(off + m0 + mr) * F + nrow] = (_Float16)swiglu(acc[mb][0][j], acc[mb][1][j]);
        }
    }
}

template <int TYPE>
__global__ void __launch_bounds__(GM_TPB)
k_grouped_down(const _Float16 *__restrict__ h16, int F, ExpertWeights ew, int N, BucketOut b,
               float *__restrict__ y)
{
    __shared__ __attribute__((aligned(16))) _Float16 As[GM_TILE_M * GM_ROW];
    const int item = blockIdx.y;
    if (item >= *b.n_tiles) return;
    const int packed = b.tiles[item];
    const int e = packed >> 16, mt = packed & 0xffff;
    const int off = b.offsets[e], c_e = b.counts[e];
    const int m0 = mt * GM_TILE_M;
    const int mrows = min(GM_TILE_M, c_e - m0);
    const int mblocks = (mrows + 15) / 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    const int arow0 = tid >> 5, achunk = tid & 31;
    int64_t row_off[GM_ACH];
#pragma unroll
    for (int i = 0; i < GM_ACH; i++) {
        const int r = arow0 + (GM_TPB / 32) * i;
        row_off[i] = r < mrows ? (int64_t)(off + m0 + r) * F : -1;
    }

    const uint8_t *wd = ebase(ew.down, ew.table, e, 2, (uint64_t)N, ew.down_stride);
    const int nrow = blockIdx.x * GM_TILE_N + 16 * wave + (lane & 15);
    const uint8_t *rows[1] = { wd + (size_t)nrow * ew.down_stride };

    floatx4 acc[4][1];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i][0] = floatx4{ 0.f, 0.f, 0.f, 0.f };

    gm_kloop_mb<TYPE, 1>(mblocks, h16, row_off, arow0, achunk, rows, F / 256, lane, As, acc);

#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int mr = 16 * mb + 4 * (lane >> 4) + j;
            if (mr < mrows) y[(int64_t)(off + m0 + mr) * N + nrow] = acc[mb][0][j];
        }
    }
}

bool grouped_type_ok(int type, int K)
{
    if (K <= 0 || K % 256 != 0) return false;
    return type == T_Q4_K || type == T_Q6_K || type == T_Q8_0 || type == T_F32;
}

#define DS3_T_SWITCH(TY, CALL)                                                  \
    switch (TY) {                                                               \
    case T_F32: { constexpr int TV = T_F32; CALL; } break;                      \
    case T_Q8_0: { constexpr int TV = T_Q8_0; CALL; } break;                    \
    case T_Q4_K: { constexpr int TV = T_Q4_K; CALL; } break;                    \
    case T_Q6_K: { constexpr int TV = T_Q6_K; CALL; } break;                    \
    default: return hipErrorInvalidValue;                                       \
    }

hipError_t launch_grouped_gate_up(const _Float16 *x16, int K, const ExpertWeights &ew, int F, const BucketOut &b,
                                  _Float16 *h16, hipStream_t s)
{
    if (ew.gate_type != ew.up_type || !grouped_type_ok(ew.gate_type, K) || F % GM_TILE_N != 0 ||
        b.tile_m != GM_TILE_M)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)(F / GM_TILE_N), (unsigned)b.max_tiles);
    DS3_T_SWITCH(ew.gate_type, hipLaunchKernelGGL((k_grouped_gate_up<TV>), grid, dim3(GM_TPB), 0, s,
                                                  x16, K, ew, F, b, h16));
    return hipGetLastError();
}

hipError_t launch_grouped_down(const _Float16 *h16, int F, const ExpertWeights &ew, int N, const BucketOut &b,
                               float *y, hipStream_t s)
{
    if (!grouped_type_ok(ew.down_type, F) || N % GM_TILE_N != 0 || b.tile_m != GM_TILE_M)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)(N / GM_TILE_N), (unsigned)b.max_tiles);
    DS3_T_SWITCH(ew.down_type, hipLaunchKernelGGL((k_grouped_down<TV>), grid, dim3(GM_TPB), 0, s,
                                                  h16, F, ew, N, b, y));
    return hipGetLastError();
}

}  // namespace ds3k
