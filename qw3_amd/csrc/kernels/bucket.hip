// bucket.hip -- token -> expert bucketing for the gathered prefill path.
//
// Same order as the reference's host loop (src/ds3_engine.c:932-955): each
// expert's list holds its tokens in increasing token order.  The rank of slot
// (t, e) inside expert e's list is the number of earlier tokens that chose e,
// read from LDS bitmaps: bit t%32 of mask[t/32][e] is set when token t chose
// e, so rank = (prefix of popcounts over earlier 32-token chunks) +
// popcount(mask & lanes-below-t).  No atomics touch the output, so the lists
// are deterministic.  One workgroup; LDS holds ceil(T/32) * E masks (u32)
// and prefixes (u16) (T <= 2560 for E = 128), and, where it also fits, the
// expert-ordered token ids (u16) and weights, which leave in one coalesced
// copy instead of as scattered 4-byte stores (10 us of the 15 us the
// scatter took at T = 2048).
//
// It also emits the grouped-GEMM work list: for each expert with c > 0
// tokens, ceil(c / tile_m) items packed as (expert << 16) | m_tile, expert
// order; experts with no tokens produce no work.  A slot whose expert id is
// outside [0, E) is dropped (slot_pos = -1) rather than trusted.
#include "common.h"
#include "launch.h"

namespace ds3k {

constexpr int BUCKET_TPB = 1024;
constexpr size_t BUCKET_MASK_BYTES = 60 * 1024;   // masks (u32) + prefix (u16)
constexpr size_t BUCKET_LDS_BYTES = 144 * 1024;   // ... + staged ids (u16) and weights (f32)

// Inclusive prefix sum over the wavefront (DPP row shifts, then rows 1 and 3
// add lane 15 of the row below, rows 2 and 3 lane 31).
__device__ __forceinline__ int wave_scan_i(int v)
{
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
    return v;
}

// Exclusive prefix sums of (a, b) over threads 0 .. n-1 (the first waves of
// the workgroup; every thread calls it); totals returned in ta, tb.
__device__ __forceinline__ void block_scan2(int &a, int &b, int &ta, int &tb, int n, int2 *wsum)
{
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int nw = (n + WAVE - 1) / WAVE;
    int ia = 0, ib = 0;
    if (wave < nw) {
        ia = wave_scan_i(a);
        ib = wave_scan_i(b);
        if (lane == WAVE - 1) wsum[wave] = make_int2(ia, ib);
    }
    __syncthreads();
    int pa = 0, pb = 0;
    ta = 0;
    tb = 0;
    for (int w = 0; w < nw; w++) {
        const int2 v = wsum[w];
        if (w < wave) { pa += v.x; pb += v.y; }
        ta += v.x;
        tb += v.y;
    }
    a = pa + ia - a;
    b = pb + ib - b;
}

// Slots per thread kept in registers between the passes: every slot of
// T <= 2560 tokens x 8 (the LDS limit above), so both passes read the routing
// once; a slot past them is re-read inside each pass's loop, where every
// iteration waits for its load.
constexpr int BUCKET_CACHE = 20;

// Word offset of the staged lists in the LDS array (after masks and prefixes).
__host__ __device__ constexpr size_t bucket_stage_words(int chunks, int E)
{
    return (size_t)chunks * E + ((size_t)chunks * E + 1) / 2;
}

// Work items and run lists (every thread of the block calls it, after the
// count scan): e = threadIdx.x, cnt = expert e's slot count, off = its first
// list position, tb = its first tile, ntile = its tiles, total_t = all
// tiles; xs: LDS scratch of BUCKET_XS_WORDS(E, max_tiles) words.  Per-expert
// tile facts go to xs: each tile's expert, each expert's first tile, offset
// and count, and for the run lists the tile counts by cost class.
__host__ __device__ constexpr int bucket_xs_words(int E, int max_tiles) { return 5 * E + (max_tiles + 1) / 2; }

__device__ void bucket_lists(int e, int cnt, int off, int tb, int ntile, int total_t, int E, const BucketOut &o,
                             int2 *wsum, uint32_t *xs)
{
    const int nt = total_t < o.max_tiles ? total_t : o.max_tiles;
    int *tb_s = (int *)xs;                        // [E] first tile of each expert
    uint32_t *info_s = xs + E;                    // [E] full tiles << 16 | m blocks of the last tile
    uint32_t *cpos_s = info_s + E;                // [E] class-4 position << 16 | last tile's class position
    int *off_s = (int *)(cpos_s + E);             // [E] first list position of each expert
    int *cnt_s = off_s + E;                       // [E] slot count of each expert
    uint16_t *own_s = (uint16_t *)(cnt_s + E);    // [nt] expert of each tile
    if (e < E) {
        tb_s[e] = tb;
        off_s[e] = off;
        cnt_s[e] = cnt;
        for (int m = 0; m < ntile && tb + m < nt; m++) own_s[tb + m] = (uint16_t)e;
    }
    const bool runs = o.runs_gu != nullptr;
    __syncthreads();                                      // wsum is read before the next scan writes it
    if (runs) {
        // run lists: (tile, n-run) for every tile, gate_up's and down's,
        // heaviest first: tiles of 4 m blocks (16-token blocks), then 3, 2, 1,
        // each class in tile order.  A run's cost grows with its m blocks,
        // and the grouped kernels deal the list out round by round, so the
        // rounds then hold runs of like cost.  Only an expert's last tile can
        // have fewer than 4 m blocks.
        const int full = cnt / o.tile_m, rest = cnt - full * o.tile_m;
        const int mb_last = rest > 0 ? (4 * rest + o.tile_m - 1) / o.tile_m : 0;   // quarters of a tile: 1 .. 4
        int a4 = e < E ? full + (mb_last == 4 ? 1 : 0) : 0, a3 = e < E && mb_last == 3 ? 1 : 0;
        int a2 = e < E && mb_last == 2 ? 1 : 0, a1 = e < E && mb_last == 1 ? 1 : 0;
        int n4 = 0, n3 = 0, n2 = 0, n1 = 0;
        block_scan2(a4, a3, n4, n3, E, wsum);
        __syncthreads();                                  // wsum is read before the next scan writes it
        block_scan2(a2, a1, n2, n1, E, wsum);
        if (e < E) {
            // position among all tiles of this expert's first class-4 tile and of its last tile
            const int last = mb_last == 4 || mb_last == 0 ? 0
                           : mb_last == 3 ? n4 + a3 : mb_last == 2 ? n4 + n3 + a2 : n4 + n3 + n2 + a1;
            info_s[e] = ((uint32_t)full << 16) | (uint32_t)mb_last;
            cpos_s[e] = ((uint32_t)a4 << 16) | (uint32_t)last;
        }
    }
    __syncthreads();
    // One thread per tile (work item) writes its work item and runs.
    for (int q = threadIdx.x; q < nt; q += BUCKET_TPB) {
        const int lo = own_s[q], m = q - tb_s[lo];
        o.tiles[q] = (lo << 16) | m;
        if (runs) {
            const uint32_t inf = info_s[lo], cp = cpos_s[lo];
            const bool c4 = m < (int)(inf >> 16) || (inf & 0xffffu) == 4u;
            const int pos = c4 ? (int)(cp >> 16) + m : (int)(cp & 0xffffu);
            if (pos < o.max_tiles) {
                // the run's descriptor: its tile's first list position and rows
                const int row0 = off_s[lo] + m * o.tile_m, mrows = min(o.tile_m, cnt_s[lo] - m * o.tile_m);
                const int dy = (lo << 16) | (mrows << 8);
                for (int j = 0; j < o.rpi_gu; j++) {
                    o.runs_gu[pos * o.rpi_gu + j] = (q << 12) | j;
                    if (o.desc_gu) o.desc_gu[pos * o.rpi_gu + j] = make_int2(row0, dy | j);
                }
                for (int j = 0; j < o.rpi_dn; j++) {
                    o.runs_dn[pos * o.rpi_dn + j] = (q << 12) | j;
                    if (o.desc_dn) o.desc_dn[pos * o.rpi_dn + j] = make_int2(row0, dy | j);
                }
            }
        }
    }
    if (runs && threadIdx.x == 0) {
        o.n_runs[0] = nt * o.rpi_gu;
        o.n_runs[1] = nt * o.rpi_dn;
    }
    __syncthreads();
}

__global__ void __launch_bounds__(BUCKET_TPB)
k_bucket(const int32_t *__restrict__ idx, const float *__restrict__ scores, int T, int k, int E, BucketOut o,
         int stage)
{
    __shared__ __attribute__((aligned(16))) uint32_t sm[BUCKET_LDS_BYTES / 4];
    const int chunks = (T + 31) / 32;
    uint32_t *mask = sm;                                  // [chunks][E]
    uint16_t *pre = (uint16_t *)(sm + chunks * E);        // [chunks][E] exclusive prefix
    float *wts_l = (float *)(sm + bucket_stage_words(chunks, E));   // stage: [T k] weights by position
    uint16_t *ids_l = (uint16_t *)(wts_l + T * k);                  //        [T k] token ids by position
    __shared__ int32_t off_s[BUCKET_TPB];
    __shared__ int2 wsum[BUCKET_TPB / WAVE];
    const int S = T * k;
    int ex_c[BUCKET_CACHE];
    float sc_c[BUCKET_CACHE];
#pragma unroll
    for (int i = 0; i < BUCKET_CACHE; i++) {             // the slots' ids and scores, loaded once
        const int s = threadIdx.x + BUCKET_TPB * i;
        ex_c[i] = s < S ? idx[s] : -1;
        sc_c[i] = s < S ? scores[s] : 0.f;
    }
    for (int i = threadIdx.x; i < chunks * E; i += BUCKET_TPB) mask[i] = 0u;
    __syncthreads();
    auto mark = [&](int s, int e) {
        const int t = s / k;
        if (e >= 0 && e < E) atomicOr(&mask[(t >> 5) * E + e], 1u << (t & 31));
    };
#pragma unroll
    for (int i = 0; i < BUCKET_CACHE; i++)
        if (threadIdx.x + BUCKET_TPB * i < S) mark(threadIdx.x + BUCKET_TPB * i, ex_c[i]);
    for (int s = threadIdx.x + BUCKET_TPB * BUCKET_CACHE; s < S; s += BUCKET_TPB) mark(s, idx[s]);
    __syncthreads();
    // Per-chunk prefixes of each expert's bits: G = BUCKET_TPB / E threads per
    // expert, thread (g, e) = g * E + e owns a run of consecutive chunks; run
    // totals meet in off_s (free until the offsets), then each thread writes
    // its run's prefixes.  Thread e then holds its expert's count.
    const int e = threadIdx.x;                            // E <= BUCKET_TPB
    {
        const int G = BUCKET_TPB / E, gi = threadIdx.x / E, ei = threadIdx.x - gi * E;
        const int L = (chunks + G - 1) / G, c0 = gi * L, c1 = min(chunks, c0 + L);
        int part = 0;
        if (gi < G)
            for (int c = c0; c < c1; c++) part += __popc(mask[c * E + ei]);
        off_s[threadIdx.x] = part;
        __syncthreads();
        if (gi < G) {
            int run = 0;
            for (int g = 0; g < gi; g++) run += off_s[g * E + ei];
            for (int c = c0; c < c1; c++) {
                pre[c * E + ei] = (uint16_t)run;
                run += __popc(mask[c * E + ei]);
            }
        }
    }
    int cnt = 0;
    if (e < E)
        for (int g = 0; g < BUCKET_TPB / E; g++) cnt += off_s[g * E + e];
    __syncthreads();                                      // off_s is read before it is rewritten
    int off = cnt, tb = (cnt + o.tile_m - 1) / o.tile_m, total = 0, total_t = 0;
    const int ntile = tb;
    block_scan2(off, tb, total, total_t, E, wsum);
    if (e < E) {
        o.counts[e] = cnt;
        o.offsets[e] = off;
        off_s[e] = off;
    }
    if (threadIdx.x == 0) {
        o.offsets[E] = total;
        *o.n_tiles = total_t < o.max_tiles ? total_t : o.max_tiles;
    }
    bucket_lists(e, cnt, off, tb, ntile, total_t, E, o, wsum, sm + bucket_stage_words(chunks, E));
    auto place = [&](int s, int ex, float sc) {
        const int t = s / k;
        if (ex < 0 || ex >= E) {          // out-of-range id: the slot is dropped
            o.slot_pos[s] = -1;
            return;
        }
        const int w = (t >> 5) * E + ex;
        const int rank = (int)pre[w] + __popc(mask[w] & ((1u << (t & 31)) - 1u));
        const int pos = off_s[ex] + rank;
        if (stage) {
            ids_l[pos] = (uint16_t)t;
            wts_l[pos] = sc;
        } else {
            o.ids[pos] = t;
            o.wts[pos] = sc;
        }
        o.slot_pos[s] = pos;
    };
#pragma unroll
    for (int i = 0; i < BUCKET_CACHE; i++)
        if (threadIdx.x + BUCKET_TPB * i < S) place(threadIdx.x + BUCKET_TPB * i, ex_c[i], sc_c[i]);
    for (int s = threadIdx.x + BUCKET_TPB * BUCKET_CACHE; s < S; s += BUCKET_TPB) place(s, idx[s], scores[s]);
    if (stage) {
        __syncthreads();
        for (int p = threadIdx.x; p < total; p += BUCKET_TPB) {   // positions 0 .. total-1 are all placed
            o.ids[p] = ids_l[p];
            o.wts[p] = wts_l[p];
        }
    }
}

// Placement from the bitmaps k_route_mark writes: bit t % 4 of
// masks[t / 4][e] is set when token t chose expert e; the 8 rows of a
// 32-token chunk make k_bucket's 32-bit bitmap of that chunk, so the lists
// come out in the same order.  Workgroup c places the slots of tokens 32c ..
// 32c+31: every workgroup sums the bit counts of all chunks per expert (the
// totals, and the part before its chunk), scans the totals for the offsets
// and writes its own slots' token ids, weights and positions; workgroup 0
// also writes counts, offsets, work items and run lists.  T <= PLACE_MAX_T,
// k <= 32, E <= PLACE_MAX_E.
constexpr int PLACE_MAX_T = 2048;
constexpr int PLACE_MAX_E = 256;
constexpr int PLACE_MAX_TILES = PLACE_MAX_T * 32 / 64 + PLACE_MAX_E;

// The 32-bit bitmap of chunk c for expert e from its 8 rows of 4-token bytes
// (rows past the last token are not read).
__device__ __forceinline__ uint32_t place_mask(const uint8_t *rowsb, int c, int e, int E, int rows)
{
    uint32_t m = 0u;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = 8 * c + i;
        if (r < rows) m |= (uint32_t)rowsb[r * E + e] << (4 * i);
    }
    return m;
}

// Copies n16 16-byte pieces of the bitmap rows into LDS, N per thread: all N
// loads are issued (a load past the last piece re-reads it and is not
// written), then the pieces are written.  N * BUCKET_TPB >= n16.
template <int N>
__device__ __forceinline__ void place_copy_rows(const uint8_t *__restrict__ masks, uint8_t *rowsb, int n16)
{
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const int i0 = threadIdx.x;
    u32x4_t v[N];
#pragma unroll
    for (int u = 0; u < N; u++) v[u] = ((const u32x4_t *)masks)[min(i0 + BUCKET_TPB * u, n16 - 1)];
    // the compiler would otherwise sink each load into its write's branch and wait there
    if constexpr (N == 2) asm volatile("" : "+v"(v[0]), "+v"(v[1]));
    if constexpr (N == 4) asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
    if constexpr (N == 8)
        asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),
                     "+v"(v[7]));
#pragma unroll
    for (int u = 0; u < N; u++)
        if (i0 + BUCKET_TPB * u < n16) ((u32x4_t *)rowsb)[i0 + BUCKET_TPB * u] = v[u];
}

__global__ void __launch_bounds__(BUCKET_TPB)
k_bucket_place(const int32_t *__restrict__ idx, const float *__restrict__ scores, const uint8_t *__restrict__ masks,
               int T, int k, int E, BucketOut o)
{
    __shared__ int32_t part_s[2][BUCKET_TPB];      // partial counts per (thread group, expert): all chunks, earlier chunks
    __shared__ int32_t off_s[PLACE_MAX_E], pre_s[PLACE_MAX_E];
    __shared__ uint32_t own_s[PLACE_MAX_E];       // this chunk's bitmaps
    __shared__ int2 wsum[BUCKET_TPB / WAVE];
    __shared__ uint32_t xs[bucket_xs_words(PLACE_MAX_E, PLACE_MAX_TILES)];
    __shared__ __attribute__((aligned(16))) uint8_t rowsb[PLACE_MAX_T / 4 * PLACE_MAX_E];   // all rows of the call
    const int c = blockIdx.x, chunks = (T + 31) / 32, rows = (T + 3) / 4;
    {
        // every row into LDS at once: 16-byte loads (masks 16-byte aligned),
        // all of a thread's loads issued before any is written, so the copy
        // is one memory round trip; the tail by bytes
        const int nb = rows * E, n16 = nb / 16;
        static_assert(8 * BUCKET_TPB * 16 >= PLACE_MAX_T / 4 * PLACE_MAX_E, "8 loads per thread cover every row");
        const int nper = (n16 + BUCKET_TPB - 1) / BUCKET_TPB;     // loads per thread, <= 8
        if (n16 <= 0) {
        } else if (nper == 1) place_copy_rows<1>(masks, rowsb, n16);
        else if (nper == 2) place_copy_rows<2>(masks, rowsb, n16);
        else if (nper <= 4) place_copy_rows<4>(masks, rowsb, n16);
        else place_copy_rows<8>(masks, rowsb, n16);
        for (int i = 16 * n16 + (int)threadIdx.x; i < nb; i += BUCKET_TPB) rowsb[i] = masks[i];
    }
    __syncthreads();
    {
        // G threads per expert, each over a run of consecutive chunks
        const int G = BUCKET_TPB / E, gi = threadIdx.x / E, ei = threadIdx.x - gi * E;
        const int L = (chunks + G - 1) / G, c0 = gi * L, c1 = min(chunks, c0 + L);
        int tot = 0, before = 0;
        if (gi < G)
            for (int cc = c0; cc < c1; cc++) {
                const int n = __popc(place_mask(rowsb, cc, ei, E, rows));
                tot += n;
                if (cc < c) before += n;
            }
        part_s[0][threadIdx.x] = tot;
        part_s[1][threadIdx.x] = before;
        if ((int)threadIdx.x < E) own_s[threadIdx.x] = place_mask(rowsb, c, threadIdx.x, E, rows);
    }
    __syncthreads();
    const int e = threadIdx.x;
    int cnt = 0, pc = 0;
    if (e < E)
        for (int g = 0; g < BUCKET_TPB / E; g++) {
            cnt += part_s[0][g * E + e];
            pc += part_s[1][g * E + e];
        }
    int off = cnt, tb = (cnt + o.tile_m - 1) / o.tile_m, total = 0, total_t = 0;
    const int ntile = tb;
    block_scan2(off, tb, total, total_t, E, wsum);
    if (e < E) {
        off_s[e] = off;
        pre_s[e] = pc;
    }
    if (c == 0) {                                         // uniform over the workgroup
        if (e < E) {
            o.counts[e] = cnt;
            o.offsets[e] = off;
        }
        if (threadIdx.x == 0) {
            o.offsets[E] = total;
            *o.n_tiles = total_t < o.max_tiles ? total_t : o.max_tiles;
        }
        bucket_lists(e, cnt, off, tb, ntile, total_t, E, o, wsum, xs);   // its barriers also publish off_s, pre_s
    } else {
        __syncthreads();
    }
    // this chunk's slots, one per thread
    const int s = c * 32 * k + (int)threadIdx.x;
    if ((int)threadIdx.x < 32 * k && s < T * k) {
        const int t = s / k, ex = idx[s];
        if (ex < 0 || ex >= E) {                          // out-of-range id: the slot is dropped
            o.slot_pos[s] = -1;
        } else {
            const int pos = off_s[ex] + pre_s[ex] + __popc(own_s[ex] & ((1u << (t & 31)) - 1u));
            o.ids[pos] = t;
            o.wts[pos] = scores[s];
            o.slot_pos[s] = pos;
        }
    }
}

hipError_t launch_bucket_place(const int32_t *idx, const float *scores, const uint8_t *masks, int T, int k, int E,
                               const BucketOut &o, hipStream_t s)
{
    if (T <= 0 || T > PLACE_MAX_T || k <= 0 || k > 32 || E <= 0 || E > PLACE_MAX_E || o.max_tiles < 0 ||
        o.max_tiles > PLACE_MAX_TILES || ((uintptr_t)masks & 15) != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_bucket_place, dim3((unsigned)((T + 31) / 32)), dim3(BUCKET_TPB), 0, s, idx, scores, masks, T,
                       k, E, o);
    return hipGetLastError();
}

// The lists of a dense product (matmul_quantized_batch on the grouped
// kernel): one expert holding rows 0 .. M-1 in order with weight 1, work
// items 0 .. nt-1, and the run lists in item order -- which is k_bucket's
// heaviest-first order here, as every tile but the last is full.
__global__ void __launch_bounds__(BUCKET_TPB) k_dense_lists(int M, BucketOut o)
{
    const int nt = (M + o.tile_m - 1) / o.tile_m;
    for (int i = threadIdx.x; i < M; i += BUCKET_TPB) {
        o.ids[i] = i;
        o.wts[i] = 1.0f;
        o.slot_pos[i] = i;
    }
    for (int q = threadIdx.x; q < nt; q += BUCKET_TPB) o.tiles[q] = q;      // expert 0, tile q
    for (int i = threadIdx.x; i < nt * o.rpi_gu; i += BUCKET_TPB) {
        const int q = i / o.rpi_gu, j = i % o.rpi_gu;
        o.runs_gu[i] = (q << 12) | j;
        if (o.desc_gu) o.desc_gu[i] = make_int2(q * o.tile_m, (min(o.tile_m, M - q * o.tile_m) << 8) | j);
    }
    if (o.runs_dn != nullptr)
        for (int i = threadIdx.x; i < nt * o.rpi_dn; i += BUCKET_TPB) {
            const int q = i / o.rpi_dn, j = i % o.rpi_dn;
            o.runs_dn[i] = (q << 12) | j;
            if (o.desc_dn) o.desc_dn[i] = make_int2(q * o.tile_m, (min(o.tile_m, M - q * o.tile_m) << 8) | j);
        }
    if (threadIdx.x == 0) {
        o.counts[0] = M;
        o.offsets[0] = 0;
        o.offsets[1] = M;
        *o.n_tiles = nt;
        o.n_runs[0] = nt * o.rpi_gu;
        o.n_runs[1] = o.runs_dn != nullptr ? nt * o.rpi_dn : 0;
    }
}

hipError_t launch_dense_lists(int M, const BucketOut &o, hipStream_t s)
{
    if (M <= 0 || o.tile_m <= 0 || o.runs_gu == nullptr || o.rpi_gu <= 0 || (M + o.tile_m - 1) / o.tile_m > o.max_tiles ||
        (M + o.tile_m - 1) / o.tile_m > 4095)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_dense_lists, dim3(1), dim3(BUCKET_TPB), 0, s, M, o);
    return hipGetLastError();
}

hipError_t launch_bucket(const int32_t *idx, const float *scores, int T, int k, int E, const BucketOut &o,
                         hipStream_t s)
{
    const int chunks = (T + 31) / 32;
    const size_t lds = (size_t)chunks * E * (sizeof(uint32_t) + sizeof(uint16_t));
    if (T <= 0 || T > 65535 || k <= 0 || E <= 0 || E > 1024 || lds > BUCKET_MASK_BYTES || o.max_tiles < 0)
        return hipErrorInvalidValue;
    // the per-expert tile facts and the tile owner table share the staging area
    if ((bucket_stage_words(chunks, E) + (size_t)bucket_xs_words(E, o.max_tiles)) * 4 > BUCKET_LDS_BYTES)
        return hipErrorInvalidValue;
    const size_t staged = bucket_stage_words(chunks, E) * 4 + (size_t)T * k * (sizeof(float) + sizeof(uint16_t));
    const int stage = staged <= BUCKET_LDS_BYTES ? 1 : 0;
    hipLaunchKernelGGL(k_bucket, dim3(1), dim3(BUCKET_TPB), 0, s, idx, scores, T, k, E, o, stage);
    return hipGetLastError();
}

}  // namespace ds3k
