// moe_decode.hip -- expert products for small token counts (decode).
//
// Bandwidth-bound GEMVs that stream each selected expert's quantised rows
// once, decoding in registers (reference decode kernels metal/moe.metal:140-391,
// host dispatch src/ds3_metal.m:2075-2290).  Two launches:
//   gate_up: h[slot][r] = silu(x_t . Wg_e[r]) * (x_t . Wu_e[r])
//   down:    out[t][j] = out[t][j] + w_0 y_0[j] + ... + w_{k-1} y_{k-1}[j]
//            with y_k[j] = h[slot_k] . Wd_{e_k}[j], summed in top-k order
//            (reference src/ds3_reference.c:674-678), no atomics.
#include "route_select.h"
#include "rowstream.h"

namespace ds3k {

__device__ __forceinline__ const uint8_t *expert_base(const uint8_t *base, const uint64_t *table, int e,
                                                      int which, uint64_t rows, uint64_t stride)
{
    return base + (table ? table[3 * e + which] : (uint64_t)e * rows * stride);
}

constexpr int DEC_TPB = 256;
static_assert(DEC_TPB == XC_THREADS, "the exact-weights stage runs on a decode workgroup's four waves");
#ifndef DS3_DOWN_PREFETCH
#ifndef DS3_DOWN_PREFETCH
#define DS3_DOWN_PREFETCH 1    // T = 1: the fused gate/up kernel warms L2 with the down rows
#endif
#endif
constexpr int N_XCD_DEC = 8;   // MI355X: workgroups go round-robin to 8 XCDs
#ifndef DS3_DOWN_LDS
#define DS3_DOWN_LDS 1         // Q6_K / Q8_0 down rows staged through LDS by DMA
#endif
#ifndef DS3_GU_CHUNKED
#define DS3_GU_CHUNKED 1       // T = 2..16 gate/up rows through the chunked row stream
#endif
#ifndef DS3_SEL_RPW
#define DS3_SEL_RPW 4          // rows per lane group in the fused-selection gate/up kernel
#endif

// PAIR: h = swiglu(gate, up).  !PAIR: h = gate projection only, with expert
// offsets from table column `which` (unfused fallback for mixed types).
// Lane group (G lanes) per row, UPL = K/32/G units per lane, RPW rows per
// group: the trip counts are compile-time and rows past F are clamped (their
// results dropped), so every load of a wave is issued before its first dot
// product and the wave pays one memory round trip.  Rows of expert e for
// routed slot `slot` (token row xt), row block rb of the expert.
template <int GT, int G, int UPL, bool PAIR, int RPW = 2>
__device__ __forceinline__ void gate_up_rows(const float *__restrict__ xt, int slot, int rb, int e,
                                             const ExpertWeights &ew, int K, int F, int which, float *__restrict__ h)
{
    constexpr int GPW = WAVE / G;
    const uint8_t *wg = expert_base(ew.gate, ew.table, e, PAIR ? 0 : which, (uint64_t)F, ew.gate_stride);
    const uint8_t *wu = PAIR ? expert_base(ew.up, ew.table, e, 1, (uint64_t)F, ew.up_stride) : wg;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int gl = lane % G, grp = lane / G;
    const int r0 = (rb * (DEC_TPB / WAVE) + wave) * GPW * RPW + grp;
    float ag[RPW], au[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const int r = min(r0 + GPW * i, F - 1);
        const uint8_t *grow = wg + (size_t)r * ew.gate_stride;
        const uint8_t *urow = wu + (size_t)r * ew.up_stride;
        ag[i] = 0.f;
        au[i] = 0.f;
        const int upl = UPL > 0 ? UPL : K / 32 / G;
#pragma unroll
        for (int j = 0; j < (UPL > 0 ? UPL : 1); j++) {
            ag[i] += unit_dot<GT>(grow, gl + G * j, xt);
            if (PAIR) au[i] += unit_dot<GT>(urow, gl + G * j, xt);
        }
        for (int j = (UPL > 0 ? UPL : 1); j < upl; j++) {   // shapes without a compile-time count
            ag[i] += unit_dot<GT>(grow, gl + G * j, xt);
            if (PAIR) au[i] += unit_dot<GT>(urow, gl + G * j, xt);
        }
    }
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const int r = r0 + GPW * i;
        const float a = group_sum<G>(ag[i]);
        const float b = PAIR ? group_sum<G>(au[i]) : 0.f;
        if (r < F && gl == 0) h[(int64_t)slot * F + r] = PAIR ? swiglu(a, b) : a;
    }
}

// One-dimensional grid: n_exact workgroups first (xt.w set: workgroup t
// recomputes token t's weights from the exact logits of its selected
// experts, exact_weights_wg, routing by k_router_select; dispatched first,
// they run beside the row workgroups), then nx row blocks per slot.
template <int GT, int G, int UPL, bool PAIR>
__global__ void __launch_bounds__(DEC_TPB)
k_decode_gate_up(const float *__restrict__ x, int64_t ldx, const int32_t *__restrict__ idx, int n_used,
                 ExpertWeights ew, int K, int F, int which, float *__restrict__ h, int nx, int n_exact, ExactTail xt)
{
    extern __shared__ __attribute__((aligned(16))) float xt_lds[];   // exact_chain_lds(K) bytes with xt.w set
    if ((int)blockIdx.x < n_exact) {
        const int t = blockIdx.x, wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
        float4 xv[4];
        exact_load_x(x + (int64_t)t * ldx, K, xv, threadIdx.x);
        const int e_lane = lane < n_used ? idx[t * n_used + lane] : 0;
        exact_store_x(xt_lds, K, xv, threadIdx.x);
        __syncthreads();                                         // the row is in LDS
        exact_weights_wg(xt_lds, K, xt.w, xt.wstride, xt.ra, t, e_lane, wave, lane);
        return;
    }
    const int r = blockIdx.x - n_exact, slot = r / nx;
    gate_up_rows<GT, G, UPL, PAIR>(x + (int64_t)(slot / n_used) * ldx, slot, r - slot * nx, idx[slot], ew, K, F,
                                   which, h);
}

// ---------------------------------------------------------------------------
// Chunked gate/up rows (T = 2..16 decode, dense Q4_K / Q6_K / Q8_0 rows of
// K = 2048 / 4096 from 16-byte aligned expert bases): workgroup w of slot s
// takes chunks c = w, w + wps, ... of DG_R consecutive gate rows and the same
// up rows, each a contiguous byte range, loaded by every thread into register
// sets (two chunks of both matrices in flight, rowstream.h) and staged in two
// LDS buffers; each wave dots DG_R / 4 rows of both with the slot's token x,
// held in registers for the workgroup's whole walk, and lane 63 writes
// h = silu(gate) * up.  Against gate_up_rows: x is read once per workgroup,
// not once per row, and the weights arrive as whole lines.  The first
// n_exact workgroups run the exact-weights stage as in k_decode_gate_up; both
// paths carve the same dynamic LDS.
// ---------------------------------------------------------------------------
#ifndef DS3_DG_ROWS
#define DS3_DG_ROWS 4
#endif
#ifndef DS3_DG_WPC
#define DS3_DG_WPC 3
#endif
constexpr int DG_R = DS3_DG_ROWS;                // rows per chunk, of gate and of up
constexpr int DG_WPC = DS3_DG_WPC;               // workgroups per CU over all slots
static_assert(DG_R >= 4 && DG_R % 4 == 0, "each of the 4 waves dots DG_R / 4 rows of a chunk");

template <int GT, int UPL>
struct DgChunk {
    static constexpr int RB = G1Row<GT>::RB * UPL;
    static constexpr int CB = DG_R * RB;
    static constexpr int NL = (CB + G1_LOAD - 1) / G1_LOAD;
    static constexpr int BUF = NL * G1_LOAD;
    static constexpr size_t LDS = (size_t)4 * BUF;   // two chunks of gate and up
    static_assert(3 * NL <= 63, "three sets in flight behind the oldest");
};

template <int GT, int UPL>
__global__ void __launch_bounds__(DEC_TPB)
k_decode_gate_up_chunked(const float *__restrict__ x, int64_t ldx, const int32_t *__restrict__ idx, int n_used,
                         ExpertWeights ew, int F, float *__restrict__ h, int wps, int nch, int n_exact, ExactTail xt)
{
    static_assert(DEC_TPB == G1_TPB, "row streaming assumes 256 threads");
    extern __shared__ __attribute__((aligned(16))) uint8_t dl[];
    constexpr int K = 2048 * UPL;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    if ((int)blockIdx.x < n_exact) {
        const int t = blockIdx.x;
        float4 xv[4];
        exact_load_x(x + (int64_t)t * ldx, K, xv, threadIdx.x);
        const int e_lane = lane < n_used ? idx[t * n_used + lane] : 0;
        exact_store_x((float *)dl, K, xv, threadIdx.x);
        __syncthreads();                                         // the row is in LDS
        exact_weights_wg((float *)dl, K, xt.w, xt.wstride, xt.ra, t, e_lane, wave, lane);
        return;
    }
    using P = DgChunk<GT, UPL>;
    const int r = (int)blockIdx.x - n_exact, slot = r / wps;
    int c = r - slot * wps;
    if (c >= nch) return;                                        // uniform over the workgroup
    const int e = idx[slot];
    const uint8_t *wg = expert_base(ew.gate, ew.table, e, 0, (uint64_t)F, ew.gate_stride);
    const uint8_t *wu = expert_base(ew.up, ew.table, e, 1, (uint64_t)F, ew.up_stride);
    const int64_t lim = (int64_t)F * P::RB - 16;
    G1Set<P::NL> SG[2], SU[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int64_t o = (int64_t)min(c + j * wps, nch - 1) * P::CB;
        SG[j].issue(wg, o, P::CB, lim);
        SU[j].issue(wu, o, P::CB, lim);
    }
    // x after the first chunks: the wait for x (vmcnt 0, in issue order)
    // then covers them too, one memory latency instead of two
    float xr[UPL][32], sx[UPL][4];
    g1_load_x<GT, UPL>(x + (int64_t)(slot / n_used) * ldx, lane, xr, sx);
    bool more = true;
    for (int k = 0; more; k += 2) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            if (more) {                                          // uniform over the workgroup
                SG[j].template wait<3 * P::NL>();                // SU[j] and the other chunk's pair went out after
                SU[j].template wait<2 * P::NL>();
                uint8_t *buf = dl + ((k + j) & 1) * 2 * P::BUF;
                SG[j].to_lds(buf);
                SU[j].to_lds(buf + P::BUF);
                __syncthreads();                                 // every wave is done with this buffer's last chunk
                const int64_t o = (int64_t)min(c + 2 * wps, nch - 1) * P::CB;
                SG[j].issue(wg, o, P::CB, lim);
                SU[j].issue(wu, o, P::CB, lim);
#pragma unroll 1
                for (int i = 0; i < DG_R / 4; i++) {
                    const int rr = wave + 4 * i;
                    float ag = 0.f, au = 0.f;
#pragma unroll
                    for (int q = 0; q < UPL; q++) {
                        ag += g1_unit_dot<GT>(buf + rr * P::RB, lane + 64 * q, xr[q], sx[q]);
                        au += g1_unit_dot<GT>(buf + P::BUF + rr * P::RB, lane + 64 * q, xr[q], sx[q]);
                    }
                    ag = g1_wave_total(ag);
                    au = g1_wave_total(au);
                    const int row = c * DG_R + rr;
                    if (lane == WAVE - 1 && row < F) h[(int64_t)slot * F + row] = swiglu(ag, au);
                }
                c += wps;
                more = c < nch;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {                                // loads still in flight, registers named
        SG[j].template wait<0>();
        SU[j].template wait<0>();
    }
}

template <int GT, int UPL>
static hipError_t gate_up_chunked_t(const float *x, int64_t ldx, const int32_t *idx, int n_slots, int n_used,
                                    const ExpertWeights &ew, int F, float *h, int n_exact, const ExactTail &tail,
                                    size_t exact_lds, hipStream_t s)
{
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    using P = DgChunk<GT, UPL>;
    const int nch = (F + DG_R - 1) / DG_R;
    // DG_WPC workgroups per CU over all slots, at least one per slot
    int wps = DG_WPC * n_cu / n_slots;
    wps = wps < 1 ? 1 : wps > nch ? nch : wps;
    const size_t lds = std::max(P::LDS, exact_lds);
    const dim3 grid((unsigned)(n_exact + (int64_t)wps * n_slots));
    hipLaunchKernelGGL((k_decode_gate_up_chunked<GT, UPL>), grid, dim3(DEC_TPB), lds, s, x, ldx, idx, n_used, ew, F,
                       h, wps, nch, n_exact, tail);
    return hipGetLastError();
}

// The chunked kernel's shapes: gate and up of one type among Q4_K / Q6_K /
// Q8_0, K = 2048 or 4096, dense rows, 16-byte aligned tensors, no offset
// table (its expert offsets are on the device, where their alignment is not
// checked).
static bool gate_up_chunked_ok(const ExpertWeights &ew, int K)
{
    if (ew.gate_type != ew.up_type || (K != 2048 && K != 4096) || ew.table != nullptr) return false;
    if (((uintptr_t)ew.gate & 15) != 0 || ((uintptr_t)ew.up & 15) != 0) return false;
    int rb;
    switch (ew.gate_type) {
    case T_Q4_K: rb = G1Row<T_Q4_K>::RB; break;
    case T_Q6_K: rb = G1Row<T_Q6_K>::RB; break;
    case T_Q8_0: rb = G1Row<T_Q8_0>::RB; break;
    default: return false;
    }
    const uint64_t row = (uint64_t)rb * (uint64_t)(K / 2048);
    return ew.gate_stride == row && ew.up_stride == row;
}

// The exact-weights stage on its own, one workgroup per token: token t's
// weights from the reference's exact logits of its selected experts (the
// routing of the certified router's selection launch), for callers that run
// no decode gate/up launch after it (the grouped prefill path).
__global__ void __launch_bounds__(DEC_TPB)
k_exact_weights(const float *__restrict__ x, int64_t ldx, ExactTail xt, int K)
{
    extern __shared__ __attribute__((aligned(16))) float xw_lds[];   // exact_chain_lds(K) bytes
    const int t = blockIdx.x, wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    float4 xv[4];
    exact_load_x(x + (int64_t)t * ldx, K, xv, threadIdx.x);
    const int e_lane = lane < xt.ra.k ? xt.ra.idx[(int64_t)t * xt.ra.out_stride + lane] : 0;
    exact_store_x(xw_lds, K, xv, threadIdx.x);
    __syncthreads();                                             // the row is in LDS
    exact_weights_wg(xw_lds, K, xt.w, xt.wstride, xt.ra, t, e_lane, wave, lane);
}

// Warm each XCD's L2 with the down rows its down workgroups will read:
// workgroups go round-robin to the 8 XCDs in dispatch order, so down
// workgroup x (rows 8x .. 8x+7 of every selected expert, one token) runs on
// XCD x % 8, as does gate/up workgroup `lin` (its linear index in a grid of
// nwg).  One dword per 64-byte line; the values are only consumed, never
// stored.  Whole 16-byte aligned 8-row blocks: every dword read lies inside
// them.  e_rank: lane r < n_used holds the expert of rank r.
__device__ __forceinline__ uint32_t prefetch_down_rows(const ExpertWeights &ew, int K, int n_used, int e_rank,
                                                       int lin, int nwg)
{
    uint32_t pf = 0u;
    if (DS3_DOWN_PREFETCH && n_used <= WAVE && K % 8 == 0 && ew.table == nullptr &&
        (8 * ew.down_stride) % 16 == 0 && ((uintptr_t)ew.down & 15) == 0) {
        const int xcd = lin % N_XCD_DEC, li = lin / N_XCD_DEC, nli = (nwg - xcd + N_XCD_DEC - 1) / N_XCD_DEC;
        const int K_rows = K, dwg = K_rows / 8;                // down: n_embd rows, 8 per workgroup
        const int pairs = (dwg - xcd + N_XCD_DEC - 1) / N_XCD_DEC * n_used;
        const int lines = (int)((8 * ew.down_stride + 63) / 64);
        for (int p = li; p < pairs; p += nli) {
            const int xd = xcd + N_XCD_DEC * (p / n_used), k = p - (p / n_used) * n_used;
            const int ek = __builtin_amdgcn_readlane(e_rank, k);
            const uint8_t *base = expert_base(ew.down, ew.table, ek, 2, (uint64_t)K_rows, ew.down_stride) +
                                  (size_t)8 * xd * ew.down_stride;
            for (int l = threadIdx.x; l < lines; l += DEC_TPB) pf ^= *(const uint32_t *)(base + 64 * (size_t)l);
        }
    }
    return pf;
}

// gate_up with the certified router's selection in its prologue: every
// wave ranks the experts of its token from the sums S / bounds B on its own
// (no LDS, no barrier on the common path) and takes the expert of its slot;
// a token it cannot certify is repaired by the whole workgroup, and wave 0
// of the token's first row block writes its routing outputs.  A certified
// token's outputs come from its exact-weights workgroup (the first T of the
// one-dimensional grid, dispatched first): it evaluates the reference's
// exact logits of the k selected experts and the weights from them
// (exact_weights_wg) while the row workgroups (nx per slot) stream the
// expert weights.  This removes the selection launch and its memory round
// trip from the decode chain.
template <int GT, int G, int UPL>
__global__ void __launch_bounds__(DEC_TPB)
k_decode_gate_up_sel(const float *__restrict__ x, int n_used, ExpertWeights ew, int K, int F,
                     float *__restrict__ h, int nx, CertSel cs, RouteArgs ra)
{
    extern __shared__ __attribute__((aligned(16))) float sel_prod[];
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
    const int lin = blockIdx.x, nwg = gridDim.x;
    int e_rank = 0;
    if ((int)blockIdx.x < ra.T) {
        const int t = blockIdx.x;
        // every wave ranks the token (the same result: an uncertified token,
        // left to the repair, leaves the whole workgroup) and stages a part
        // of its row
        float4 xv[4];
        exact_load_x(x + (int64_t)t * K, K, xv, threadIdx.x);
        const bool ok = cert_select_wave(cs.ca, ra, t, false, lane, e_rank);
        if (!ok) return;
        exact_store_x(sel_prod, K, xv, threadIdx.x);
        __syncthreads();                                         // the row is in LDS
        exact_weights_wg(sel_prod, K, cs.w, cs.wstride, ra, t, e_rank, wave, lane);
        if (wave == 0 && lane == 0 && cs.ca.stats != nullptr) atomicAdd(&cs.ca.stats[0], 1ull);
        return;
    }
    const int r = blockIdx.x - ra.T, slot = r / nx, rb = r - slot * nx;
    const int t = slot / n_used, kk = slot - t * n_used;
    // One wave ranks the token and hands the ranking to the others through
    // LDS (the selection is a few hundred VALU instructions: repeated by
    // every wave it cost more issue time than the rows' dot products).  The
    // selecting wave rotates with the workgroup, so the selections of a CU's
    // workgroups fall on different SIMDs.
    __shared__ int sel_s[1 + WAVE];                           // certified flag, then the experts by rank
    if (wave == (int)(blockIdx.x & (DEC_TPB / WAVE - 1))) {
        const bool ok = cert_select_wave(cs.ca, ra, t, false, lane, e_rank);
        if (lane == 0) sel_s[0] = ok ? 1 : 0;
        if (ok && lane < n_used) sel_s[1 + lane] = e_rank;
    }
    const bool emit = rb == 0 && kk == 0;
    __syncthreads();
    const bool certified = sel_s[0] != 0;                     // uniform: the general path needs every wave
    if (certified) e_rank = lane < n_used ? sel_s[1 + lane] : 0;
    const int e = certified ? sel_s[1 + kk]
                            : cert_select_tokens<1>(x, K, cs.w, cs.wstride, cs.ca, ra, t, emit, sel_prod)[kk];
    const uint32_t pf = certified ? prefetch_down_rows(ew, K, n_used, e_rank, lin, nwg) : 0u;
    gate_up_rows<GT, G, UPL, true, DS3_SEL_RPW>(x + (int64_t)t * K, slot, rb, e, ew, K, F, 0, h);
    asm volatile("" ::"v"(pf));                // the prefetch loads stay
}

// One wave per selected expert k, lane group (G lanes) per output row, UPL
// units per lane with compile-time trip counts (all loads issued first).
template <int DT, int G, int UPL>
__global__ void __launch_bounds__(1024)
k_decode_down(const float *__restrict__ h, const int32_t *__restrict__ idx, const float *__restrict__ wts,
              int n_used, ExpertWeights ew, int N, int F, int rows_per_wg, float *__restrict__ out,
              int64_t ldo, const float *__restrict__ residual, int accumulate)
{
    extern __shared__ float part[];            // [n_used][rows_per_wg]
    const int t = blockIdx.y;
    const int k = threadIdx.x / WAVE;          // one wave per selected expert
    const int slot = t * n_used + k;
    const int e = idx[slot];
    const uint8_t *wd = expert_base(ew.down, ew.table, e, 2, (uint64_t)N, ew.down_stride);
    const float *hs = h + (int64_t)slot * F;

    const int lane = threadIdx.x & (WAVE - 1);
    const int gl = lane % G, grp = lane / G;  // rows_per_wg == WAVE / G: one row per group
    const int j = min(blockIdx.x * rows_per_wg + grp, N - 1);
    const uint8_t *row = wd + (size_t)j * ew.down_stride;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < (UPL > 0 ? UPL : 1); i++) acc += unit_dot<DT>(row, gl + G * i, hs);
    for (int i = (UPL > 0 ? UPL : 1); i < F / 32 / G; i++) acc += unit_dot<DT>(row, gl + G * i, hs);
    acc = group_sum<G>(acc);
    if (gl == 0) part[k * rows_per_wg + grp] = acc;
    __syncthreads();
    for (int rr = threadIdx.x; rr < rows_per_wg; rr += blockDim.x) {
        const int jj = blockIdx.x * rows_per_wg + rr;
        if (jj >= N) continue;
        float *o = out + (int64_t)t * ldo + jj;
        {
#pragma clang fp contract(off)
            float a = accumulate ? *o : 0.0f;
            for (int kk = 0; kk < n_used; kk++) a = a + wts[t * n_used + kk] * part[kk * rows_per_wg + rr];
            if (residual) a = a + residual[(int64_t)t * ldo + jj];
            *o = a;
        }
    }
}

// ---------------------------------------------------------------------------
// Q6_K and Q8_0 down with the weights staged through LDS.  Same work split
// and the same arithmetic as k_decode_down<DT, 8, UPL> (so the same results,
// bit for bit): wave k of the workgroup is slot k, lane group (8 lanes) per
// row, 8 rows per wave, UPL = F / 256 units of 32 weights per lane.  The
// wave's 8 rows are contiguous (8 x 210 UPL or 8 x 272 UPL bytes, a multiple
// of 16) and arrive by 16-byte global_load_lds DMAs together with the slot's
// h row, so a lane's unit fields (runs at 2-byte offsets: dword reads and
// funnel shifts) and its h come from LDS instead of ~20-40 small global
// loads.  N % 8 == 0, F % 256 == 0 with F <= 1024, rows packed, 16-byte
// aligned expert bases and h.
// ---------------------------------------------------------------------------
#define DS3_LDSP __attribute__((address_space(3)))

__device__ __forceinline__ uint2 lds_u64_a2(uint32_t a)
{
    const DS3_LDSP uint32_t *q = (const DS3_LDSP uint32_t *)(uintptr_t)(a & ~3u);
    const uint32_t sh = a & 3u;
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

// unit_dot_q6k with the row's block and x in LDS (byte addresses)
__device__ __forceinline__ float unit_dot_q6k_lds(uint32_t row, int u, uint32_t xa)
{
    const int b = u >> 3, h = (u >> 2) & 1, j = u & 3;
    const uint32_t blk = row + (uint32_t)b * 210u;
    const uint2 lo = lds_u64_a2(blk + 64 * h + 8 * j);
    const uint2 hi = lds_u64_a2(blk + 64 * h + 32 + 8 * j);
    const uint2 qh = lds_u64_a2(blk + 128 + 32 * h + 8 * j);
    const uint2 scw = lds_u64_a2(blk + 192 + 8 * h);       // scales[8h .. 8h+7]
    const float d = h2f(*(const DS3_LDSP uint16_t *)(uintptr_t)(blk + 208));
    const int s0 = j >> 1;                                  // group (8j)/16 within the half
    const DS3_LDSP float *xb = (const DS3_LDSP float *)(uintptr_t)xa + 256 * b + 128 * h + 8 * j;
    const uint32_t low[2] = { lo.x, lo.y }, hig[2] = { hi.x, hi.y }, hb[2] = { qh.x, qh.y };
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t sc_byte = byte_of(t < 2 ? scw.x : scw.y, (s0 + 2 * t) & 3);
        const float sc = (float)(int8_t)sc_byte;
        const DS3_LDSP float *xt = xb + 32 * t;
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

__device__ __forceinline__ uint32_t lds_u32_a2(uint32_t a)
{
    const DS3_LDSP uint32_t *q = (const DS3_LDSP uint32_t *)(uintptr_t)(a & ~3u);
    return __builtin_amdgcn_alignbyte(q[1], q[0], a & 3u);
}

// unit_dot_q80 with the row's block and x in LDS (byte addresses): the same
// operations in the same order
__device__ __forceinline__ float unit_dot_q80_lds(uint32_t row, int u, uint32_t xa)
{
    const uint32_t blk = row + (uint32_t)u * 34u;
    const float d = h2f(*(const DS3_LDSP uint16_t *)(uintptr_t)blk);
    const DS3_LDSP float *xb = (const DS3_LDSP float *)(uintptr_t)xa + 32 * u;
    float dc = 0.f, sx = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t q = lds_u32_a2(blk + 2 + 4 * i) ^ 0x80808080u;   // int8 + 128
        dc += dot4(q, xb + 4 * i);
        sx += sum4(xb + 4 * i);
    }
    return d * (dc - 128.f * sx);
}

// Bytes of one down row of F = 256 UPL weights.
template <int DT> struct DownRow;
template <> struct DownRow<T_Q6_K> { static constexpr int PER256 = 210; };
template <> struct DownRow<T_Q8_0> { static constexpr int PER256 = 272; };

template <int DT, int UPL>
__global__ void __launch_bounds__(1024)
k_decode_down_lds(const float *__restrict__ h, const int32_t *__restrict__ idx, const float *__restrict__ wts,
                  int n_used, ExpertWeights ew, int N, int F, float *__restrict__ out, int64_t ldo,
                  const float *__restrict__ residual, int accumulate)
{
    constexpr int G = 8, RPW = WAVE / G, ROWB = DownRow<DT>::PER256 * UPL;
    constexpr int WB = RPW * ROWB, REGION = WB + 1024 * UPL;   // 8 rows, then h (F = 256 UPL floats)
    extern __shared__ __attribute__((aligned(16))) uint8_t dsm[];
    const int t = blockIdx.y;
    const int k = threadIdx.x / WAVE;          // one wave per selected expert
    const int lane = threadIdx.x & (WAVE - 1);
    const int slot = t * n_used + k;
    const int e = idx[slot];
    const int j0 = blockIdx.x * RPW;
    const uint8_t *src = expert_base(ew.down, ew.table, e, 2, (uint64_t)N, ew.down_stride) + (size_t)j0 * ROWB;
    const float *hs = h + (int64_t)slot * F;
    const uint32_t reg = (uint32_t)(uintptr_t)(DS3_LDSP void *)dsm + (uint32_t)(k * REGION);
    // rows: WB / 16 chunks, 64 per instruction (the last one partly masked); h: 64 UPL chunks
#pragma unroll
    for (int i = 0; i < (WB / 16 + WAVE - 1) / WAVE; i++) {
        const int c = WAVE * i + lane;
        if (c < WB / 16)
            __builtin_amdgcn_global_load_lds(src + 16 * c, (DS3_LDSP void *)(uintptr_t)(reg + 1024u * i), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < UPL; i++)
        __builtin_amdgcn_global_load_lds(hs + 256 * i + 4 * lane, (DS3_LDSP void *)(uintptr_t)(reg + WB + 1024u * i),
                                         16, 0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's rows and h are in LDS (its own region)
    const int gl = lane % G, grp = lane / G;
    const uint32_t row = reg + (uint32_t)(grp * ROWB);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        if constexpr (DT == T_Q6_K) acc += unit_dot_q6k_lds(row, gl + G * i, reg + WB);
        else acc += unit_dot_q80_lds(row, gl + G * i, reg + WB);
    }
    acc = group_sum<G>(acc);
    float *part = (float *)(dsm + n_used * REGION);        // [n_used][RPW]
    if (gl == 0) part[k * RPW + grp] = acc;
    __syncthreads();
    for (int rr = threadIdx.x; rr < RPW; rr += blockDim.x) {
        const int jj = j0 + rr;
        float *o = out + (int64_t)t * ldo + jj;
        {
#pragma clang fp contract(off)
            float a = accumulate ? *o : 0.0f;
            for (int kk = 0; kk < n_used; kk++) a = a + wts[t * n_used + kk] * part[kk * RPW + rr];
            if (residual) a = a + residual[(int64_t)t * ldo + jj];
            *o = a;
        }
    }
}

// Lanes per row: the largest power of two <= 64 dividing the row's units.
static int lanes_per_row(int units)
{
    int g = 1;
    while (g < 64 && units % (2 * g) == 0) g *= 2;
    return g;
}

#define DS3_G_SWITCH(G, CALL)                                                   \
    switch (G) {                                                                \
    case 1: { constexpr int GV = 1; CALL; } break;                              \
    case 2: { constexpr int GV = 2; CALL; } break;                              \
    case 4: { constexpr int GV = 4; CALL; } break;                              \
    case 8: { constexpr int GV = 8; CALL; } break;                              \
    case 16: { constexpr int GV = 16; CALL; } break;                            \
    case 32: { constexpr int GV = 32; CALL; } break;                            \
    case 64: { constexpr int GV = 64; CALL; } break;                            \
    default: return hipErrorInvalidValue;                                       \
    }

// Units per lane as a compile-time count for the shapes of the configs
// (1: K = 2048 at 64 lanes, 3: K = 768 at 8 lanes); 0 = runtime loop.
#define DS3_U_SWITCH(U, CALL)                                                   \
    switch (U) {                                                                \
    case 1: { constexpr int UV = 1; CALL; } break;                              \
    case 3: { constexpr int UV = 3; CALL; } break;                              \
    default: { constexpr int UV = 0; CALL; } break;                             \
    }

#define DS3_T_SWITCH(TY, CALL)                                                  \
    switch (TY) {                                                               \
    case T_F32: { constexpr int TV = T_F32; CALL; } break;                      \
    case T_Q8_0: { constexpr int TV = T_Q8_0; CALL; } break;                    \
    case T_Q4_K: { constexpr int TV = T_Q4_K; CALL; } break;                    \
    case T_Q6_K: { constexpr int TV = T_Q6_K; CALL; } break;                    \
    default: return hipErrorInvalidValue;                                       \
    }


static bool exact_tail_ok(const ExactTail *xt, int n_slots, int n_used, int K)
{
    return xt->ra.k == n_used && xt->ra.T * n_used == n_slots && xt->ra.idx != nullptr && xt->ra.scores != nullptr &&
           xt->ra.logits != nullptr && xt->ra.out_stride == n_used && router_cert_ok(K, xt->ra.E, n_used) &&
           ((uintptr_t)xt->w & 15) == 0 && xt->wstride % 4 == 0;
}

static hipError_t decode_gate_up_impl(const float *x, int64_t ldx, const int32_t *idx, int n_slots, int n_used,
                                      const ExpertWeights &ew, int K, int F, float *h, bool pair, int which,
                                      const ExactTail *xt, hipStream_t s)
{
    if (!gemv_type_ok(ew.gate_type, K) || n_slots <= 0 || F <= 0) return hipErrorInvalidValue;
    if (xt != nullptr && (!exact_tail_ok(xt, n_slots, n_used, K) || idx != xt->ra.idx || ldx % 4 != 0 ||
                          ((uintptr_t)x & 15) != 0))
        return hipErrorInvalidValue;
    const ExactTail tail = xt != nullptr ? *xt : ExactTail{};
    const size_t lds = xt != nullptr ? exact_chain_lds(K) : 0;
    if (pair && DS3_GU_CHUNKED && gate_up_chunked_ok(ew, K)) {
        const int n_exact = xt != nullptr ? xt->ra.T : 0;
        const bool two = K == 4096;
        switch (ew.gate_type) {
        case T_Q4_K:
            return two ? gate_up_chunked_t<T_Q4_K, 2>(x, ldx, idx, n_slots, n_used, ew, F, h, n_exact, tail, lds, s)
                       : gate_up_chunked_t<T_Q4_K, 1>(x, ldx, idx, n_slots, n_used, ew, F, h, n_exact, tail, lds, s);
        case T_Q6_K:
            return two ? gate_up_chunked_t<T_Q6_K, 2>(x, ldx, idx, n_slots, n_used, ew, F, h, n_exact, tail, lds, s)
                       : gate_up_chunked_t<T_Q6_K, 1>(x, ldx, idx, n_slots, n_used, ew, F, h, n_exact, tail, lds, s);
        default:
            return two ? gate_up_chunked_t<T_Q8_0, 2>(x, ldx, idx, n_slots, n_used, ew, F, h, n_exact, tail, lds, s)
                       : gate_up_chunked_t<T_Q8_0, 1>(x, ldx, idx, n_slots, n_used, ew, F, h, n_exact, tail, lds, s);
        }
    }
    const int G = lanes_per_row(K / 32), UPL = K / 32 / G;
    const int rows_per_wg = (DEC_TPB / WAVE) * (WAVE / G) * 2;     // 2 rows per lane group
    const int nx = (F + rows_per_wg - 1) / rows_per_wg, n_exact = xt != nullptr ? xt->ra.T : 0;
    const dim3 grid((unsigned)(n_exact + (int64_t)nx * n_slots));
    if (pair) {
        DS3_T_SWITCH(ew.gate_type, DS3_G_SWITCH(G, DS3_U_SWITCH(UPL, hipLaunchKernelGGL(
            (k_decode_gate_up<TV, GV, UV, true>), grid, dim3(DEC_TPB), lds, s, x, ldx, idx, n_used, ew, K, F, which, h,
            nx, n_exact, tail))));
    } else {
        DS3_T_SWITCH(ew.gate_type, DS3_G_SWITCH(G, DS3_U_SWITCH(UPL, hipLaunchKernelGGL(
            (k_decode_gate_up<TV, GV, UV, false>), grid, dim3(DEC_TPB), lds, s, x, ldx, idx, n_used, ew, K, F, which, h,
            nx, n_exact, tail))));
    }
    return hipGetLastError();
}

hipError_t launch_decode_gate_up(const float *x, int64_t ldx, const int32_t *idx, int n_slots, int n_used,
                                 const ExpertWeights &ew, int K, int F, float *h, hipStream_t s, const ExactTail *xt)
{
    if (ew.gate_type != ew.up_type) return hipErrorInvalidValue;
    return decode_gate_up_impl(x, ldx, idx, n_slots, n_used, ew, K, F, h, true, 0, xt, s);
}

hipError_t launch_decode_gate_up_sel(const float *x, int T, int n_used, const ExpertWeights &ew, int K, int F,
                                     float *h, const CertSel &cs, const RouteArgs &ra, hipStream_t s)
{
    if (ew.gate_type != ew.up_type || !gemv_type_ok(ew.gate_type, K) || T <= 0 || F <= 0 || ra.T != T ||
        ra.k != n_used || ra.idx == nullptr || ra.scores == nullptr || !router_cert_ok(K, ra.E, n_used))
        return hipErrorInvalidValue;
    const int G = lanes_per_row(K / 32), UPL = K / 32 / G;
    const int rows_per_wg = (DEC_TPB / WAVE) * (WAVE / G) * DS3_SEL_RPW;
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)cs.w & 15) != 0 || cs.wstride % 4 != 0 || ra.out_stride != n_used ||
        ra.logits == nullptr)
        return hipErrorInvalidValue;
    // T exact-weights workgroups, then nx row blocks per slot
    const int nx = (F + rows_per_wg - 1) / rows_per_wg;
    const dim3 grid((unsigned)(T + (int64_t)nx * T * n_used));
    const size_t lds = std::max((size_t)cs.ca.nb * (K + 4) * sizeof(float), exact_chain_lds(K));
    DS3_T_SWITCH(ew.gate_type, DS3_G_SWITCH(G, DS3_U_SWITCH(UPL, hipLaunchKernelGGL(
        (k_decode_gate_up_sel<TV, GV, UV>), grid, dim3(DEC_TPB), lds, s, x, n_used, ew, K, F, h, nx, cs, ra))));
    return hipGetLastError();
}

hipError_t launch_exact_weights(const float *x, int64_t ldx, const ExactTail &xt, int K, hipStream_t s)
{
    if (xt.w == nullptr || xt.ra.T <= 0 || !exact_tail_ok(&xt, xt.ra.T * xt.ra.k, xt.ra.k, K) || ldx % 4 != 0 ||
        ((uintptr_t)x & 15) != 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_exact_weights, dim3((unsigned)xt.ra.T), dim3(DEC_TPB), exact_chain_lds(K), s, x, ldx, xt, K);
    return hipGetLastError();
}

hipError_t launch_decode_proj(const float *x, int64_t ldx, const int32_t *idx, int n_slots, int n_used,
                              const ExpertWeights &ew, int which, int K, int F, float *out, hipStream_t s,
                              const ExactTail *xt)
{
    return decode_gate_up_impl(x, ldx, idx, n_slots, n_used, ew, K, F, out, false, which, xt, s);
}

hipError_t launch_decode_down(const float *h, const int32_t *idx, const float *wts, int T, int n_used,
                              const ExpertWeights &ew, int N, int F, float *out, int64_t ldo,
                              const float *residual, bool accumulate, hipStream_t s)
{
    if (!gemv_type_ok(ew.down_type, F) || T <= 0 || N <= 0 || n_used <= 0 || n_used > 16)
        return hipErrorInvalidValue;
    const int per256 = ew.down_type == T_Q6_K ? 210 : 272;
    if (DS3_DOWN_LDS && (ew.down_type == T_Q6_K || ew.down_type == T_Q8_0) && N % 8 == 0 && F % 256 == 0 &&
        F <= 1024 && ew.down_stride == (uint64_t)(per256 * (F / 256)) && ((uintptr_t)ew.down & 15) == 0 &&
        (ew.table == nullptr) && ((uintptr_t)h & 15) == 0) {
        const int upl = F / 256;
        const size_t lds = (size_t)n_used * (8 * per256 * upl + 1024 * upl) + (size_t)n_used * 8 * sizeof(float);
        const dim3 grid((unsigned)(N / 8), (unsigned)T);
#define DS3_DLDS(DTV, U) hipLaunchKernelGGL((k_decode_down_lds<DTV, U>), grid, dim3(n_used * WAVE), lds, s, h, idx, \
                                           wts, n_used, ew, N, F, out, ldo, residual, accumulate ? 1 : 0)
        if (lds <= 163840) {
            if (ew.down_type == T_Q6_K) switch (upl) {
            case 1: DS3_DLDS(T_Q6_K, 1); break;
            case 2: DS3_DLDS(T_Q6_K, 2); break;
            case 3: DS3_DLDS(T_Q6_K, 3); break;
            default: DS3_DLDS(T_Q6_K, 4); break;
            }
            else switch (upl) {
            case 1: DS3_DLDS(T_Q8_0, 1); break;
            case 2: DS3_DLDS(T_Q8_0, 2); break;
            case 3: DS3_DLDS(T_Q8_0, 3); break;
            default: DS3_DLDS(T_Q8_0, 4); break;
            }
            return hipGetLastError();
        }
#undef DS3_DLDS
    }
    const int G = lanes_per_row(F / 32), UPL = F / 32 / G;
    const int rpw = WAVE / G;                   // one row per lane group
    const dim3 grid((unsigned)((N + rpw - 1) / rpw), (unsigned)T);
    const size_t lds = (size_t)n_used * rpw * sizeof(float);
    DS3_T_SWITCH(ew.down_type, DS3_G_SWITCH(G, DS3_U_SWITCH(UPL, hipLaunchKernelGGL(
        (k_decode_down<TV, GV, UV>), grid, dim3(n_used * WAVE), lds, s, h, idx, wts, n_used, ew, N, F, rpw, out, ldo,
        residual, accumulate ? 1 : 0))));
    return hipGetLastError();
}

}  // namespace ds3k
