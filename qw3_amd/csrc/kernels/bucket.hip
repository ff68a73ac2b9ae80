// bucket.hip -- token -> expert bucketing for the gathered prefill path.
//
// Same order as the reference's host loop (src/ds3_engine.c:932-955): each
// expert's list holds its tokens in increasing token order.  The rank of slot
// (t, e) inside expert e's list is the number of earlier tokens that chose e,
// read from LDS bitmaps: bit t%32 of mask[t/32][e] is set when token t chose
// e, so rank = (prefix of popcounts over earlier 32-token chunks) +
// popcount(mask & lanes-below-t).  No atomics touch the output, so the lists
// are deterministic.  One workgroup; LDS holds ceil(T/32) * E masks (u32)
// and prefixes (u16), at most 60 KiB (T <= 2560 for E = 128).
//
// It also emits the grouped-GEMM work list: for each expert with c > 0
// tokens, ceil(c / tile_m) items packed as (expert << 16) | m_tile, expert
// order; experts with no tokens produce no work.  A slot whose expert id is
// outside [0, E) is dropped (slot_pos = -1) rather than trusted.
#include "common.h"
#include "launch.h"

namespace ds3k {

constexpr int BUCKET_TPB = 1024;
constexpr size_t BUCKET_LDS_BYTES = 60 * 1024;   // masks (u32) + prefix (u16)

__global__ void __launch_bounds__(BUCKET_TPB)
k_bucket(const int32_t *__restrict__ idx, const float *__restrict__ scores, int T, int k, int E, BucketOut o)
{
    extern __shared__ uint32_t sm[];
    const int chunks = (T + 31) / 32;
    uint32_t *mask = sm;                                  // [chunks][E]
    uint16_t *pre = (uint16_t *)(sm + chunks * E);        // [chunks][E] exclusive prefix
    __shared__ int32_t off_s[1025];
    const int S = T * k;
    for (int i = threadIdx.x; i < chunks * E; i += BUCKET_TPB) mask[i] = 0u;
    __syncthreads();
    for (int s = threadIdx.x; s < S; s += BUCKET_TPB) {
        const int t = s / k, e = idx[s];
        if (e >= 0 && e < E) atomicOr(&mask[(t >> 5) * E + e], 1u << (t & 31));
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += BUCKET_TPB) {
        int run = 0;
        for (int c = 0; c < chunks; c++) {
            pre[c * E + e] = (uint16_t)run;
            run += __popc(mask[c * E + e]);
        }
        o.counts[e] = run;
        off_s[e] = run;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0, nt = 0;
        for (int e = 0; e < E; e++) {
            const int c = off_s[e];
            off_s[e] = run;
            o.offsets[e] = run;
            for (int m = 0; m * o.tile_m < c; m++)
                if (nt < o.max_tiles) o.tiles[nt++] = (e << 16) | m;
            run += c;
        }
        off_s[E] = run;
        o.offsets[E] = run;
        *o.n_tiles = nt;
    }
    __syncthreads();
    for (int s = threadIdx.x; s < S; s += BUCKET_TPB) {
        const int t = s / k, e = idx[s];
        if (e < 0 || e >= E) {            // out-of-range id: the slot is dropped
            o.slot_pos[s] = -1;
            continue;
        }
        const int w = (t >> 5) * E + e;
        const int rank = (int)pre[w] + __popc(mask[w] & ((1u << (t & 31)) - 1u));
        const int pos = off_s[e] + rank;
        o.ids[pos] = t;
        o.wts[pos] = scores[s];
        o.slot_pos[s] = pos;
    }
}

hipError_t launch_bucket(const int32_t *idx, const float *scores, int T, int k, int E, const BucketOut &o,
                         hipStream_t s)
{
    const int chunks = (T + 31) / 32;
    const size_t lds = (size_t)chunks * E * (sizeof(uint32_t) + sizeof(uint16_t));
    if (T <= 0 || T > 65535 || k <= 0 || E <= 0 || E > 1024 || lds > BUCKET_LDS_BYTES)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_bucket, dim3(1), dim3(BUCKET_TPB), lds, s, idx, scores, T, k, E, o);
    return hipGetLastError();
}

}  // namespace ds3k
