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
// fp32 in v_mfma_f32_16x16x32_f16.  Weights are dequantised exactly in fp32
// and rounded once to fp16.
//
// Work decomposition: blockIdx.y = work item (expert, 64-token tile) from the
// bucketing kernel, blockIdx.x = 128-row output tile.  Each of the 4 waves
// owns 32 output rows (2 MFMA column blocks; gate and up both for gate_up),
// keeps their dequantised weight fragments in registers and applies them to
// all 16-token row blocks of the tile, which sit in LDS as fp16.  Per 256-wide
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
constexpr int GM_TPB = 256;
constexpr int GM_ROW = 256 + 8;           // halves per LDS row (16-byte pad)
constexpr int GM_TILE_N = 128;

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

__device__ __forceinline__ half8 to_half8(const float *w)
{
    half8 r;
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = (_Float16)w[i];
    return r;
}

__device__ __forceinline__ const uint8_t *ebase(const uint8_t *base, const uint64_t *table, int e, int which,
                                                uint64_t rows, uint64_t stride)
{
    return base + (table ? table[3 * e + which] : (uint64_t)e * rows * stride);
}

// Stage A rows [m][256 s .. 256 s + 255] of the tile: 64 rows x 32 chunks of
// 16 bytes, 8 chunks per thread.  Rows beyond the tile are zero.
struct ATile {
    uint4 r[8];
};

__device__ __forceinline__ void a_load(ATile &a, const _Float16 *src, const int64_t (&row_off)[8], int s, int chunk)
{
#pragma unroll
    for (int i = 0; i < 8; i++) {
        if (row_off[i] >= 0) a.r[i] = *(const uint4 *)(src + row_off[i] + 256 * s + 8 * chunk);
        else a.r[i] = make_uint4(0u, 0u, 0u, 0u);
    }
}

__device__ __forceinline__ void a_store(const ATile &a, _Float16 *As, int row0, int chunk)
{
#pragma unroll
    for (int i = 0; i < 8; i++) *(uint4 *)(As + (row0 + 8 * i) * GM_ROW + 8 * chunk) = a.r[i];
}

// NB column blocks of 16 rows per wave; `pairs` = gate/up (NB = 4: g0 g1 u0 u1)
// or down (NB = 2).
template <int TYPE, int NB>
__device__ __forceinline__ void gm_core(const _Float16 *As, const uint8_t *const (&rows)[NB], int s, int lane,
                                        int mblocks, floatx4 (&acc)[4][NB])
{
    const int g = lane >> 4, m = lane & 15;
#pragma unroll
    for (int hv = 0; hv < 2; hv++) {
        half8 bq[NB][4];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            float w[32];
            int k0[4];
            unit_decode<TYPE>(rows[nb], 8 * s + g + 4 * hv, w, k0);
#pragma unroll
            for (int p = 0; p < 4; p++) bq[nb][p] = to_half8(w + 8 * p);
        }
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int col = slot_k0<TYPE>(s, g, 4 * hv + p) - 256 * s;
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                if (mb < mblocks) {
                    const half8 a = *(const half8 *)(As + (16 * mb + m) * GM_ROW + col);
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[nb][p], acc[mb][nb], 0, 0, 0);
                }
            }
        }
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

    // A staging: thread covers rows (tid>>5) + 8i, 16-byte chunk tid&31.
    const int arow0 = tid >> 5, achunk = tid & 31;
    int64_t row_off[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = arow0 + 8 * i;
        row_off[i] = r < mrows ? (int64_t)b.ids[off + m0 + r] * K : -1;
    }

    const uint8_t *wg = ebase(ew.gate, ew.table, e, 0, (uint64_t)F, ew.gate_stride);
    const uint8_t *wu = ebase(ew.up, ew.table, e, 1, (uint64_t)F, ew.up_stride);
    const int nrow = blockIdx.x * GM_TILE_N + 32 * wave + (lane & 15);
    const uint8_t *rows[4] = { wg + (size_t)nrow * ew.gate_stride, wg + (size_t)(nrow + 16) * ew.gate_stride,
                               wu + (size_t)nrow * ew.up_stride, wu + (size_t)(nrow + 16) * ew.up_stride };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };

    const int S = K / 256;
    ATile a;
    a_load(a, x16, row_off, 0, achunk);
    for (int s = 0; s < S; s++) {
        __syncthreads();
        a_store(a, As, arow0, achunk);
        __syncthreads();
        if (s + 1 < S) a_load(a, x16, row_off, s + 1, achunk);
        gm_core<TYPE, 4>(As, rows, s, lane, mblocks, acc);
    }

    // Epilogue: lane holds rows 4*(lane>>4)+j of each 16-row block, column lane&15.
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int mr = 16 * mb + 4 * (lane >> 4) + j;
            if (mr < mrows) {
                _Float16 *dst = h16 + (int64_t)(off + m0 + mr) * F + nrow;
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
                    dst[16 * nb] = (_Float16)swiglu(acc[mb][nb][j], acc[mb][nb + 2][j]);
            }
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
    int64_t row_off[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = arow0 + 8 * i;
        row_off[i] = r < mrows ? (int64_t)(off + m0 + r) * F : -1;
    }

    const uint8_t *wd = ebase(ew.down, ew.table, e, 2, (uint64_t)N, ew.down_stride);
    const int nrow = blockIdx.x * GM_TILE_N + 32 * wave + (lane & 15);
    const uint8_t *rows[2] = { wd + (size_t)nrow * ew.down_stride, wd + (size_t)(nrow + 16) * ew.down_stride };

    floatx4 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = floatx4{ 0.f, 0.f, 0.f, 0.f };

    const int S = F / 256;
    ATile a;
    a_load(a, h16, row_off, 0, achunk);
    for (int s = 0; s < S; s++) {
        __syncthreads();
        a_store(a, As, arow0, achunk);
        __syncthreads();
        if (s + 1 < S) a_load(a, h16, row_off, s + 1, achunk);
        gm_core<TYPE, 2>(As, rows, s, lane, mblocks, acc);
    }

#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int mr = 16 * mb + 4 * (lane >> 4) + j;
            if (mr < mrows) {
                float *dst = y + (int64_t)(off + m0 + mr) * N + nrow;
#pragma unroll
                for (int nb = 0; nb < 2; nb++) dst[16 * nb] = acc[mb][nb][j];
            }
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
