// launch.h -- host-side launchers of the gfx950 kernels (internal interface
// between the C-ABI layer ds3_hip.cpp and the kernel translation units).
// Every launcher enqueues on `s` and returns hipGetLastError().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ds3k {

// GGUF type ids (reference src/ds3.h:201-216).
enum : int { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

// Where the three expert matrices of expert e start: either e * rows * stride
// or, if `table` is non-null, table[3e + {0,1,2}] (gate, up, down) bytes.
struct ExpertWeights {
    const uint8_t *gate, *up, *down;    // base of each packed [n_expert][rows][..] tensor
    uint64_t gate_stride, up_stride, down_stride;   // bytes per row
    int gate_type, up_type, down_type;
    const uint64_t *table;              // optional device [n_expert][3] byte offsets
};

hipError_t launch_dequant(int type, const void *src, float *dst, int64_t n, hipStream_t s);

// C[m][n] = sum_k A[m*lda + k] * W(row n)[k], W rows at w + n*stride, fp32
// accumulate.  If wnorm2 != nullptr also writes sum_k W[n][k]^2 to wnorm2[n].
hipError_t launch_gemv(int type, const float *A, int64_t lda, const uint8_t *w, uint64_t stride,
                       float *C, int64_t ldc, int M, int N, int K, float *wnorm2, hipStream_t s);

bool gemv_type_ok(int type, int K);
// Whether launch_gemv takes its one-token chunked path (k_gemv1) for these
// arguments: M = 1, Q4_K / Q6_K / Q8_0, K = 2048 or 4096, dense rows, w
// 16-byte aligned, no wnorm2.
bool gemv1_path(int type, const uint8_t *w, uint64_t stride, int M, int K);

// Router tail: logits [T][E] -> softmax -> top-k -> renorm, selected by
// (prob desc, index asc) like the reference.
struct RouteArgs {
    const float *logits;
    int32_t *idx;
    float *scores;
    int T, E, k;
    int64_t logit_stride;      // floats between tokens' logit rows
    int64_t out_stride;        // int32/float entries between tokens' idx/scores rows
    bool norm;
};
hipError_t launch_route(const RouteArgs &a, hipStream_t s);
// launch_route plus the bucketing bitmaps of launch_bucket_place: bit t % 4
// of masks[t / 4][e] (rows of E bytes) is set when token t chose expert e.
// E <= 256, k <= 32.
hipError_t launch_route_mark(const RouteArgs &a, uint8_t *masks, hipStream_t s);

// Router logits in the reference's order: logits[t][e] (row stride ldl) =
// x[t][0]*W[e][0] + x[t][1]*W[e][1] + ... summed left to right with every
// product and sum rounded to fp32, bit-identical to the reference's.  Router
// rows of any supported type (F32 / F16 / Q8_0 / Q4_K / Q6_K) at rw, rstride
// bytes apart; rows other than 4-byte aligned F32 are first expanded into
// wf32 [E][K].  If x16 != nullptr also x16[t][k] = (fp16) x[t][k].  E <= 256;
// K a whole number of blocks of rtype.  With topk (describing these logits)
// and tickets (zeroed device ints, left zeroed) the kernel may also run the
// router tail for small T; *topk_done says whether it did.
bool router_seq_type_ok(int rtype, int K);
// FP32 copy of E router rows (of type rtype, K weights each, rstride bytes
// apart) as the reference's dequantised router holds them, into dst [E][K].
hipError_t launch_router_rows(int rtype, const uint8_t *rw, uint64_t rstride, int E, int K, float *dst, hipStream_t s);
hipError_t launch_router_seq(const float *x, int T, int K, int E, int rtype, const uint8_t *rw, uint64_t rstride,
                             float *wf32, float *logits, int64_t ldl, _Float16 *x16, const RouteArgs *topk,
                             int *tickets, bool *topk_done, hipStream_t s);

// Certified router for few tokens (two launches): fp64 wavefront sums of the
// reference's fp32 products with a proven bound on the reference's
// sequential-sum error, then a selection that certifies the top-k order
// against the bounds; tokens it cannot certify get the exact sequential
// logits of their candidate experts before selection.  Indices equal the
// reference's; logits are fl32 of the fp64 sums (the exact chains for
// repaired candidates).  ra must describe these logits; scratch:
// router_cert_scratch(T, E) bytes, 8-byte aligned; x, x16 16-byte aligned.
// stats (optional): device counters {tokens certified, tokens repaired}.
// phases: bit 0 enqueues the sums (after the FP32 row copy of a non-F32
// router), bit 1 the selection; the same arguments go to both.
// norm (optional, phase 1 only with it): x holds raw rows and the sums run on
// rms_norm(x) * norm->w, the values launch_rms_norm computes, bit for bit;
// the expert-0 workgroups write them to norm->xn [T][K], which the selection
// phase (and a fused selection) then reads in place of x.  norm->w and
// norm->xn 16-byte aligned.
struct NormPro {
    const float *w;
    float eps;
    float *xn;
};
bool router_cert_ok(int K, int E, int k);
size_t router_cert_scratch(int T, int E);
hipError_t launch_router_cert(const float *x, int T, int K, int E, int rtype, const uint8_t *rw, uint64_t rstride,
                              float *wf32, float *logits, int64_t ldl, _Float16 *x16, const RouteArgs &ra,
                              void *scratch, unsigned long long *stats, int phases, hipStream_t s,
                              const NormPro *norm = nullptr);

// What the certified router's selection reads, for a kernel that selects in
// its own prologue (launch_decode_gate_up_sel) after launch_router_cert's
// phase 1 with the same arguments: the sums S and bounds B in scratch, the
// bound factor, the repair batch (nb rows of K + 4 floats) and the FP32
// router rows the sums were taken over.
struct CertArgs {
    double *S;                   // [T][E]
    float *B;                    // [T][E]
    float bfac;
    int nb;                      // candidate rows per repair batch (dynamic LDS rows of K + 4 floats)
    unsigned long long *stats;   // optional [2]: tokens certified, tokens repaired
};
struct CertSel {
    CertArgs ca;
    const float *w;              // FP32 router rows, wstride floats apart
    int64_t wstride;
};
hipError_t router_cert_sel(int T, int K, int E, int k, int rtype, const uint8_t *rw, uint64_t rstride, float *wf32,
                           void *scratch, unsigned long long *stats, int nb, CertSel *out);

// Weights of tokens routed by the certified router (k_router_select) from
// the exact logits of their selected experts, computed by a column of
// workgroups appended to the decode gate/up launch: w = the FP32 router rows
// the selection used, ra = the routing (idx / scores rows of n_used entries,
// the logits rows, whose selected entries become exact).
struct ExactTail {
    const float *w;
    int64_t wstride;
    RouteArgs ra;
};

// The same exact weights as a launch of its own (one workgroup per token of
// xt.ra), for tokens routed by the certified selection launch that no decode
// gate/up launch follows; x: the rows the router summed, ldx floats apart,
// 16-byte aligned.
hipError_t launch_exact_weights(const float *x, int64_t ldx, const ExactTail &xt, int K, hipStream_t s);

// Decode (small T) expert products.
//   h[slot][F] = silu(x[t] . Wg_e) * (x[t] . Wu_e), slot = t*n_used + k, e = idx[slot]
// With xt, also the exact weights of the tokens (xt->ra.idx == idx).
hipError_t launch_decode_gate_up(const float *x, int64_t ldx, const int32_t *idx, int n_slots,
                                 int n_used, const ExpertWeights &ew, int K, int F,
                                 float *h, hipStream_t s, const ExactTail *xt = nullptr);
// The same for the T tokens of x (rows K floats apart), with the expert of
// each slot chosen in the kernel by the certified router's selection over
// cs (launch_router_cert phase 1 done); writes ra.idx / ra.scores (and
// repaired logits) as the selection launch would, the weights of certified
// tokens from the exact logits of their selected experts (which replace
// those entries of the logits rows).
hipError_t launch_decode_gate_up_sel(const float *x, int T, int n_used, const ExpertWeights &ew, int K, int F,
                                     float *h, const CertSel &cs, const RouteArgs &ra, hipStream_t s);
//   out[slot][F] = x[t] . W_e with W = ew.gate / gate_type / gate_stride and
//   expert offsets from table column `which` (0 gate, 1 up).
hipError_t launch_decode_proj(const float *x, int64_t ldx, const int32_t *idx, int n_slots, int n_used,
                              const ExpertWeights &ew, int which, int K, int F, float *out, hipStream_t s,
                              const ExactTail *xt = nullptr);
//   out[t][j] (+)= sum_k w[t][k] * (h[slot] . Wd_e[j]) in k order
hipError_t launch_decode_down(const float *h, const int32_t *idx, const float *wts, int T,
                              int n_used, const ExpertWeights &ew, int K, int F,
                              float *out, int64_t ldo, const float *residual, bool accumulate,
                              hipStream_t s);

// Bucketing of T*n_used slots by expert, token order within each expert.
struct BucketOut {
    int32_t *counts;     // [E]
    int32_t *offsets;    // [E+1]
    int32_t *ids;        // [T*k] token of each compacted position
    float *wts;          // [T*k] routing weight of each position
    int32_t *slot_pos;   // [T*k] position of slot t*k+j
    int32_t *tiles;      // [max_tiles] packed (expert << 16 | m_tile) work items for the GEMMs
    int32_t *n_tiles;    // [1]
    int max_tiles;
    int tile_m;
    // Optional run lists of the grouped kernels (null: not written): runs
    // (tile, n-run) packed tile << 12 | n_run, in tile order.
    int32_t *runs_gu;    // [max_tiles * rpi_gu]
    int32_t *runs_dn;    // [max_tiles * rpi_dn]
    int32_t *n_runs;     // [2]: gate_up runs, down runs
    int rpi_gu, rpi_dn;  // n-runs per token tile (n tiles / n tiles per run)
    // Optional descriptors of the same runs, entry for entry (null: not
    // written): { first list position of the run's tile, expert << 16 |
    // tile rows << 8 | n run }, so a grouped kernel starts a run from one load.
    int2 *desc_gu;       // [max_tiles * rpi_gu]
    int2 *desc_dn;       // [max_tiles * rpi_dn]
};
hipError_t launch_bucket(const int32_t *idx, const float *scores, int T, int k, int E,
                         const BucketOut &o, hipStream_t s);
// The same lists from launch_route_mark's bitmaps (the rows of these T
// tokens), one workgroup per 32 tokens.  T <= 2048, k <= 32, E <= 256,
// max_tiles <= 1280.
// The lists of a dense product: one expert holding rows 0 .. M-1, in order.
hipError_t launch_dense_lists(int M, const BucketOut &o, hipStream_t s);
hipError_t launch_bucket_place(const int32_t *idx, const float *scores, const uint8_t *masks, int T, int k, int E,
                               const BucketOut &o, hipStream_t s);

// Prefill grouped products (fp16 MFMA, fp32 accumulate).
hipError_t launch_to_f16(const float *x, _Float16 *y, int64_t n, hipStream_t s);
hipError_t launch_to_f32(const _Float16 *x, float *y, int64_t n, hipStream_t s);
hipError_t launch_grouped_gate_up(const _Float16 *x16, int K, const ExpertWeights &ew, int F,
                                  const BucketOut &b, _Float16 *h16, hipStream_t s);
hipError_t launch_grouped_down(const _Float16 *h16, int F, const ExpertWeights &ew, int N,
                               const BucketOut &b, _Float16 *y, hipStream_t s);
bool grouped_type_ok(int type, int K);
// Layer shapes the grouped kernels take: n_embd a multiple of 256 x gate_up's
// weight ring depth (512 as built: whole activation chunks and ring turns per
// n tile), n_ff a multiple of 128 and at most 1024 (down's token tile stays
// in LDS).
bool grouped_shape_ok(int n_embd, int n_ff);
// Compute units of the current device (queried once; 256 if the query fails).
int device_cu_count();
// Runs per work item of the grouped kernels for a call of S slots over E
// experts (gate_up's run length depends on how many runs the call makes).
void grouped_runs_per_tile(int n_embd, int n_ff, int S, int E, int &rpi_gu, int &rpi_dn);

// Dense C[M][N] = A W^T (fp16 operands, fp32 accumulate) on the grouped
// gate_up kernel: x16 = A [M][K] in fp16; b = the bucketing lists of one
// expert holding rows 0 .. M-1 (launch_bucket of M zero indices, k = 1,
// E = 1, dense_runs_per_tile(N) gate_up runs per token tile); W rows stride
// bytes apart.  Shapes: dense_mfma_shape_ok.
bool dense_mfma_shape_ok(int type, int N, int K);
int dense_runs_per_tile(int N);
hipError_t launch_dense_mfma(const _Float16 *x16, int K, const uint8_t *w, uint64_t stride, int type, int N,
                             const BucketOut &b, float *c, hipStream_t s);

// out[t][j] = (accumulate ? out : 0) + sum_k w[t][k] * y[slot_pos[t*k+kk]][j] (+ residual)
hipError_t launch_combine(const _Float16 *y, const int32_t *slot_pos, const float *wts, int T, int k,
                          int N, float *out, int64_t ldo, const float *residual, bool accumulate,
                          hipStream_t s);

// RMSNorm of n_rows rows of n floats (row strides ldx, ldo):
// out = x * (1 / sqrt(mean(x^2) + eps)) * w (reference src/ds3_reference.c:329-342).
hipError_t launch_rms_norm(const float *x, const float *w, float *out, int n, int n_rows, float eps, int64_t ldx,
                           int64_t ldo, hipStream_t s);

// Elementwise helpers (reference metal/elementwise.metal, metal/moe.metal:95-127).
hipError_t launch_fill_zero(float *p, int64_t n, hipStream_t s);
hipError_t launch_copy(const float *a, float *b, int64_t n, hipStream_t s);
// One wave that waits `us` microseconds (at most one second) on the GPU.
hipError_t launch_hold(double us, hipStream_t s);
hipError_t launch_add(const float *a, const float *b, float *c, int64_t n, hipStream_t s);
// Row ids outside [0, n_rows) are skipped.
hipError_t launch_gather_rows(const float *src, const int32_t *ids, float *dst, int n_cols, int count,
                              int64_t n_rows, hipStream_t s);
hipError_t launch_scatter_add(const float *src, const float *scores, const int32_t *ids, float *dst,
                              int n_cols, int count, int64_t n_rows, hipStream_t s);
hipError_t launch_silu_mul(const float *g, const float *u, float *out, int64_t n, hipStream_t s);
hipError_t launch_axpy(const float *x, float w, float *y, int64_t n, hipStream_t s);

}  // namespace ds3k
