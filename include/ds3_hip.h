/*
 * ds3_hip.h -- MI355X (gfx950) backend for the qw3 MoE-FFN path.
 *
 * A C ABI that replaces the MoE subset of the reference's Metal backend
 * (reference src/ds3_metal.h).  Every ds3_metal_* entry point the engine calls
 * on this path has a ds3_hip_* counterpart with the same argument order,
 * argument meaning, return convention (0 ok, -1 error with a diagnostic on
 * stderr) and accumulate/zeroing rules; the citation on each declaration names
 * the reference declaration it replaces.  ds3_metal_compat.h maps the
 * ds3_metal_* names onto these for source-level drop-in.
 *
 * Differences a caller can observe:
 *   - Routing (softmax, top-k, renormalisation) runs on the device; nothing is
 *     read back to the host.  gate_logits still receives the router logits.
 *   - The expert_up / expert_down / hidden scratch arguments are validated as
 *     in the reference but not used: the library keeps its own device
 *     workspace.
 *   - ds3_hip_buffer_from_mmap copies the host bytes into device memory once
 *     (the MI355X is a discrete device); the buffer stays read-only.
 *   - moe_router_topk_batch_tokens writes [n_layers][n_tokens][n_used] as its
 *     documentation states (the Metal kernel's stride is only right for
 *     n_layers == 1).
 *
 * Threading: one global device context and stream, as in the reference; not
 * thread-safe.  Outside begin_batch/end_batch every call is synchronous;
 * inside, calls are enqueued on the library stream and end_batch waits.
 */
#ifndef DS3_HIP_H
#define DS3_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids: the values of the reference's ds3_type_t
 * (reference src/ds3.h:201-216).  Passed as plain int32. */
typedef int32_t ds3_hip_type_t;
#define DS3_HIP_TYPE_F32  0
#define DS3_HIP_TYPE_F16  1
#define DS3_HIP_TYPE_Q8_0 8
#define DS3_HIP_TYPE_Q4_K 12
#define DS3_HIP_TYPE_Q6_K 14

/* Opaque device buffer (reference src/ds3_metal.h:14). */
typedef struct ds3_hip_buffer ds3_hip_buffer_t;

/* ---------------------------------------------------------------------- */
/* Lifecycle and buffers                                                  */
/* ---------------------------------------------------------------------- */

/* reference src/ds3_metal.h:19-20 */
int  ds3_hip_init(void);
void ds3_hip_shutdown(void);

/* reference src/ds3_metal.h:25-26.  NULL on failure or bytes == 0. */
ds3_hip_buffer_t *ds3_hip_buffer_alloc(size_t bytes);
void              ds3_hip_buffer_free(ds3_hip_buffer_t *buf);

/* reference src/ds3_metal.h:31.  base must be page-aligned; its bytes are
 * copied to the device; the buffer refuses writes. */
ds3_hip_buffer_t *ds3_hip_buffer_from_mmap(const void *base, size_t bytes);

/* reference src/ds3_metal.h:35-36.  Shares the parent's memory. */
ds3_hip_buffer_t *ds3_hip_buffer_view(const ds3_hip_buffer_t *base, size_t offset, size_t bytes);

/* reference src/ds3_metal.h:39-42 */
int ds3_hip_buffer_write(ds3_hip_buffer_t *buf, size_t offset, const void *src, size_t bytes);
int ds3_hip_buffer_read(ds3_hip_buffer_t *buf, size_t offset, void *dst, size_t bytes);

/* ---------------------------------------------------------------------- */
/* Products with (quantised) weights                                      */
/* ---------------------------------------------------------------------- */

/* reference src/ds3_metal.h:90-94: y[out] = W[out][in] . x, F32 W */
int ds3_hip_vec_matmul_f32(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                           uint32_t in_dim, uint32_t out_dim, uint64_t row_stride);

/* reference src/ds3_metal.h:102-107: Q4_K / Q6_K / Q8_0 W */
int ds3_hip_vec_matmul_quantized(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                 uint32_t in_dim, uint32_t out_dim, uint64_t row_stride, ds3_hip_type_t type);

/* reference src/ds3_metal.h:115-137 (SIMD-group variants; same results) */
int ds3_hip_vec_matmul_f32_simd(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                uint32_t in_dim, uint32_t out_dim, uint64_t row_stride);
int ds3_hip_vec_matmul_q8_0_simd(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                 uint32_t in_dim, uint32_t out_dim, uint64_t row_stride);
int ds3_hip_vec_matmul_q4k_simd(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                uint32_t in_dim, uint32_t out_dim, uint64_t row_stride);
int ds3_hip_vec_matmul_q6k_simd(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                uint32_t in_dim, uint32_t out_dim, uint64_t row_stride);

/* reference src/ds3_metal.h:142-146: Q4_K product with an fp16 input vector
 * x[in_dim] (widened exactly to fp32), y[out_dim] fp32. */
int ds3_hip_vec_matmul_q4k_half(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                uint32_t in_dim, uint32_t out_dim, uint64_t row_stride);

/* reference src/ds3_metal.h:154-161: C[M][N] = A[M][K] . W[N][K]^T, fp32,
 * W at byte weight_offset inside the buffer.  Below the dense-MFMA row
 * count (ds3_hip_set_dense_mfma_min_rows, default 64) every product is an
 * fp32 FMA on the exactly decoded weights, as the reference's kernel
 * computes.  From that many rows, for Q4_K / Q6_K / Q8_0 with K a multiple of
 * 512 and N a multiple of 256 (the engine's prefill projections), the
 * product runs on the matrix cores with fp16 operands (A and the decoded
 * weights rounded to fp16, fp32 accumulation), the precision of the MoE
 * grouped products: relative L2 error ~5e-4 against fp32. */
int ds3_hip_matmul_quantized_batch(const ds3_hip_buffer_t *A, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *C,
                                   uint32_t M, uint32_t N, uint32_t K, uint64_t weight_row_stride,
                                   uint64_t weight_offset, ds3_hip_type_t type);

/* ---------------------------------------------------------------------- */
/* Elementwise                                                            */
/* ---------------------------------------------------------------------- */

/* reference src/ds3_metal.h:168-178 */
int ds3_hip_buffer_copy_f32(const ds3_hip_buffer_t *src, ds3_hip_buffer_t *dst, size_t bytes);
int ds3_hip_buffer_zero_f32(ds3_hip_buffer_t *buf, size_t bytes);
int ds3_hip_vec_add_inplace(ds3_hip_buffer_t *acc, const ds3_hip_buffer_t *addend, uint32_t n);
int ds3_hip_vec_add(const ds3_hip_buffer_t *a, const ds3_hip_buffer_t *b, ds3_hip_buffer_t *c, uint32_t n);

/* reference src/ds3_metal.h:184-192:
 *   gather : dst[i][j]  = src[ids[offset+i]][j]
 *   scatter: dst[ids[offset+i]][j] += scores[offset+i] * src[i][j] */
int ds3_hip_gather_rows_f32(const ds3_hip_buffer_t *src, const ds3_hip_buffer_t *ids, ds3_hip_buffer_t *dst,
                            uint32_t n_cols, uint32_t count, uint32_t offset);
int ds3_hip_scatter_add_weighted_f32(const ds3_hip_buffer_t *src, const ds3_hip_buffer_t *scores,
                                     const ds3_hip_buffer_t *ids, ds3_hip_buffer_t *dst,
                                     uint32_t n_cols, uint32_t count, uint32_t offset);

/* reference src/ds3_metal.h:195-198: out[i] = silu(gate[i]) * up[i] */
int ds3_hip_silu_mul_f32(const ds3_hip_buffer_t *gate, const ds3_hip_buffer_t *up, ds3_hip_buffer_t *out,
                         uint32_t n);

/* reference src/ds3_metal.h:48-57 (the FFN block's prologue, src/ds3_engine.c:522):
 * out[r] = x[r] / sqrt(mean(x[r]^2) + eps) * weight for n_rows rows of n.
 * The reference's formula; the sum of squares is a fixed-order tree, so the
 * result can differ from the CPU reference's left-to-right sum in the last
 * bits (as the reference's own Metal kernel's does). */
int ds3_hip_rms_norm(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *weight, ds3_hip_buffer_t *out,
                     uint32_t n, uint32_t n_rows, float eps);

/* ---------------------------------------------------------------------- */
/* MoE FFN                                                                */
/* ---------------------------------------------------------------------- */

/* reference src/ds3_metal.h:340-374 (one token).  output accumulates
 * (caller zeroes it).  expert_offsets: optional [n_expert][3] uint64 byte
 * offsets {gate, up, down}; when NULL expert e starts at e*rows*row_stride.
 * Routing uses the certified router (see ds3_hip_set_router_mode): the
 * selected experts are the reference's; gate_logits are within a proven
 * bound of the reference's sequential fp32 sums. */
int ds3_hip_moe_ffn(
    const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp,
    const ds3_hip_buffer_t *w_gate_exps, const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps,
    ds3_hip_type_t gate_type, ds3_hip_type_t up_type, ds3_hip_type_t down_type,
    uint64_t gate_row_stride, uint64_t up_row_stride, uint64_t down_row_stride,
    const ds3_hip_buffer_t *w_shared_gate, const ds3_hip_buffer_t *w_shared_up, const ds3_hip_buffer_t *w_shared_down,
    ds3_hip_type_t shared_gate_type, ds3_hip_type_t shared_up_type, ds3_hip_type_t shared_down_type,
    uint64_t shared_gate_row_stride, uint64_t shared_up_row_stride, uint64_t shared_down_row_stride,
    ds3_hip_buffer_t *output, ds3_hip_buffer_t *gate_logits, const ds3_hip_buffer_t *expert_offsets,
    ds3_hip_buffer_t *hidden, ds3_hip_buffer_t *expert_up, ds3_hip_buffer_t *expert_down,
    uint32_t n_embd, uint32_t n_expert, uint32_t n_used, uint32_t n_ff_exp, uint32_t n_ff_shared,
    uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob);

/* reference src/ds3_metal.h:380-387: gate_logits = router . input */
int ds3_hip_moe_ffn_router(const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp,
                           ds3_hip_buffer_t *gate_logits, uint32_t n_embd, uint32_t n_expert,
                           uint64_t router_row_stride, ds3_hip_type_t router_type);

/* reference src/ds3_metal.h:389-418: shared + host-selected experts */
int ds3_hip_moe_ffn_experts(
    const ds3_hip_buffer_t *input,
    const ds3_hip_buffer_t *w_gate_exps, const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps,
    ds3_hip_type_t gate_type, ds3_hip_type_t up_type, ds3_hip_type_t down_type,
    uint64_t gate_row_stride, uint64_t up_row_stride, uint64_t down_row_stride,
    const ds3_hip_buffer_t *w_shared_gate, const ds3_hip_buffer_t *w_shared_up, const ds3_hip_buffer_t *w_shared_down,
    ds3_hip_type_t shared_gate_type, ds3_hip_type_t shared_up_type, ds3_hip_type_t shared_down_type,
    uint64_t shared_gate_row_stride, uint64_t shared_up_row_stride, uint64_t shared_down_row_stride,
    ds3_hip_buffer_t *output, ds3_hip_buffer_t *hidden, ds3_hip_buffer_t *expert_up, ds3_hip_buffer_t *expert_down,
    uint32_t n_embd, uint32_t n_used, uint32_t n_ff_exp, uint32_t n_ff_shared,
    const int32_t *indices_host, const float *scores_host);

/* reference src/ds3_metal.h:424-431: logits [L][E] -> indices/scores [L][k] */
int ds3_hip_moe_router_topk_batch(const ds3_hip_buffer_t *logits, ds3_hip_buffer_t *indices,
                                  ds3_hip_buffer_t *scores, uint32_t n_layers, uint32_t n_expert,
                                  uint32_t n_used, bool norm_topk_prob);

/* reference src/ds3_metal.h:437-445: logits [L][T][E] -> [L][T][k] */
int ds3_hip_moe_router_topk_batch_tokens(const ds3_hip_buffer_t *logits, ds3_hip_buffer_t *indices,
                                         ds3_hip_buffer_t *scores, uint32_t n_layers, uint32_t n_tokens,
                                         uint32_t n_expert, uint32_t n_used, bool norm_topk_prob);

/* ---------------------------------------------------------------------- */
/* Batching and profiling                                                 */
/* ---------------------------------------------------------------------- */

/* reference src/ds3_metal.h:457-462 */
int  ds3_hip_begin_batch(void);
void ds3_hip_end_batch(void);
void ds3_hip_synchronize(void);

/* reference src/ds3_metal.h:467-468 (enabled by DS3_HIP_PROFILE=1) */
void ds3_hip_profile_reset(void);
void ds3_hip_profile_print(const char *label);

/* ---------------------------------------------------------------------- */
/* Device-routed extensions (no ds3_metal.h counterpart)                  */
/* ---------------------------------------------------------------------- */

/* The whole MoE FFN for T tokens with no host round trip: router logits,
 * softmax/top-k/renorm, then either per-token expert GEMVs (T at most the
 * crossover, see ds3_hip_set_prefill_min_tokens) or bucketing + grouped
 * fp16-MFMA products + in-order combine.  Replaces the engine's decode and
 * gathered-prefill sequences (reference src/ds3_engine.c:520-597, 895-1022).
 *   input [T][n_embd] f32; output [T][n_embd] f32 accumulates (caller
 *   zeroes); residual (optional) [T][n_embd] is added to output; output
 *   may be input itself (input += MoE(input), in place, no residual);
 *   indices / scores (optional) receive the routing [T][n_used];
 *   gate_logits (optional) receives the logits [T][n_expert].
 * The grouped products take fp16 operands (x, decoded weights, h) and keep
 * the down outputs in fp16 before the fp32 combine: outputs within rel-L2
 * 1e-3 of the fp32 reference; the per-token GEMVs are fp32 throughout.
 * Up to 16 tokens (see ds3_hip_set_router_mode) the router is the certified
 * one: indices equal the reference's; gate_logits hold the fp32 rounding of
 * the exact sum of the reference's fp32 products (the reference's own
 * sequential sums for experts whose order needed them), within a proven
 * bound of the reference's logits. */
int ds3_hip_moe_ffn_batch(
    const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp,
    const ds3_hip_buffer_t *w_gate_exps, const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps,
    ds3_hip_type_t gate_type, ds3_hip_type_t up_type, ds3_hip_type_t down_type,
    uint64_t gate_row_stride, uint64_t up_row_stride, uint64_t down_row_stride,
    const ds3_hip_buffer_t *expert_offsets,
    ds3_hip_buffer_t *output, const ds3_hip_buffer_t *residual,
    ds3_hip_buffer_t *gate_logits, ds3_hip_buffer_t *indices, ds3_hip_buffer_t *scores,
    uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert, uint32_t n_used, uint32_t n_ff_exp,
    uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob);

/* The engine's whole FFN block for T tokens in one call (reference
 * src/ds3_engine.c:519-527 and 675-720: rms_norm, zeroing, moe_ffn and the
 * residual vec_add): hidden[t] += MoE(rms_norm(hidden[t]) * ffn_norm), in
 * place.  The normalised rows go to x_norm when given (it must not overlap
 * hidden), else to the library's workspace; everything else as
 * ds3_hip_moe_ffn_batch with input = the normalised rows, output = hidden
 * (accumulating) and no separate residual.  No counterpart in ds3_metal.h. */
int ds3_hip_moe_block(
    ds3_hip_buffer_t *hidden, const ds3_hip_buffer_t *ffn_norm, float eps, const ds3_hip_buffer_t *w_gate_inp,
    const ds3_hip_buffer_t *w_gate_exps, const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps,
    ds3_hip_type_t gate_type, ds3_hip_type_t up_type, ds3_hip_type_t down_type,
    uint64_t gate_row_stride, uint64_t up_row_stride, uint64_t down_row_stride,
    const ds3_hip_buffer_t *expert_offsets, ds3_hip_buffer_t *x_norm,
    ds3_hip_buffer_t *gate_logits, ds3_hip_buffer_t *indices, ds3_hip_buffer_t *scores,
    uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert, uint32_t n_used, uint32_t n_ff_exp,
    uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob);

/* ds3_hip_moe_ffn_batch that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, semantics and results as ds3_hip_moe_ffn_batch; every
 * intermediate (routing rows, bucketing lists, h, y) lives in one library-owned
 * scratch array of ds3_hip_noalloc_scratch_bytes() bytes per GPU (64 MiB: a
 * Qwen3-30B-A3B layer call of up to 1,284 tokens), held until the process ends.
 * A call whose intermediates do not fit returns -1 with a diagnostic; split it
 * into fewer tokens.  ds3_hip_init must have been called.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (from several host
 * threads, or a graph replay with an eager call of this entry point on another
 * stream) race.  The array keeps the last call's contents; no kernel reads a
 * byte of it before the same call has written it. */
int ds3_hip_moe_ffn_batch_noalloc(
    const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp,
    const ds3_hip_buffer_t *w_gate_exps, const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps,
    ds3_hip_type_t gate_type, ds3_hip_type_t up_type, ds3_hip_type_t down_type,
    uint64_t gate_row_stride, uint64_t up_row_stride, uint64_t down_row_stride,
    const ds3_hip_buffer_t *expert_offsets,
    ds3_hip_buffer_t *output, const ds3_hip_buffer_t *residual,
    ds3_hip_buffer_t *gate_logits, ds3_hip_buffer_t *indices, ds3_hip_buffer_t *scores,
    uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert, uint32_t n_used, uint32_t n_ff_exp,
    uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob);
size_t ds3_hip_noalloc_scratch_bytes(void);

/* Router only, for T tokens: logits (bit-identical to the reference's
 * sequential fp32 sums), then indices/scores [T][n_used]. */
int ds3_hip_moe_route(const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp,
                      ds3_hip_buffer_t *gate_logits, ds3_hip_buffer_t *indices, ds3_hip_buffer_t *scores,
                      uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert, uint32_t n_used,
                      uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob);

/* Bucketing of routed slots (reference src/ds3_engine.c:932-955, compacted):
 * counts [n_expert], offsets [n_expert+1], ids/wts/slot_pos [T*n_used]. */
int ds3_hip_moe_bucket(const ds3_hip_buffer_t *indices, const ds3_hip_buffer_t *scores,
                       uint32_t n_tokens, uint32_t n_used, uint32_t n_expert,
                       ds3_hip_buffer_t *counts, ds3_hip_buffer_t *offsets, ds3_hip_buffer_t *ids,
                       ds3_hip_buffer_t *wts, ds3_hip_buffer_t *slot_pos);

/* Dequantise n values of `type` from src (byte offset src_offset) to f32 dst
 * (the parity probe for the block decoders). */
int ds3_hip_dequantize(const ds3_hip_buffer_t *src, uint64_t src_offset, ds3_hip_type_t type, uint64_t n,
                       ds3_hip_buffer_t *dst);

/* Router selection.  0 (default): the certified router (fp64 wavefront sums
 * with a proven error bound, exact sequential sums only where the bound
 * cannot certify the top-k order) in ds3_hip_moe_ffn and, up to 16 tokens,
 * in ds3_hip_moe_ffn_batch; the reference's sequential-order sums (logits
 * bit-identical to the reference's) everywhere else.  1: sequential-order
 * sums everywhere.  2: the certified router wherever its shape limits allow
 * (n_embd a multiple of 256 up to 4096), ds3_hip_moe_route included.
 * Returns the previous mode. */
int ds3_hip_set_router_mode(int mode);

/* Tokens the certified router has certified / repaired (exact sequential
 * sums for some candidates) since init or the last reset; synchronises. */
int ds3_hip_router_stats(uint64_t *certified, uint64_t *repaired, int reset);

/* Test hook (no ds3_metal.h counterpart): the bucketing lists the grouped
 * path of ds3_hip_moe_ffn_batch / _noalloc / ds3_hip_moe_block built on the
 * device for the last chunk of its last call -- the lists the reference's
 * host loop builds (src/ds3_engine.c:932-965) plus the grouped kernels' work
 * items and run lists.  Call it before any other library call that may reuse
 * the workspace; synchronises.  meta[DS3_HIP_LISTS_META] = { chunk's first
 * token, chunk's tokens tc, n_used k, n_expert E, work items n_tiles,
 * gate_up runs, down runs, 1 if the lists came from the routing's bitmaps
 * (else from the routed indices), gate_up runs per work item, down runs per
 * work item, max work items, tokens per work item }.  Each array not NULL
 * receives: counts[E], offsets[E + 1], ids / wts / slot_pos[tc * k],
 * tiles[n_tiles], runs_gu / runs_dn[their counts].  Work item = expert << 16
 * | token tile; run = work item index << 12 | n run.  -1 when no grouped call
 * ran since the workspace last moved. */
#define DS3_HIP_LISTS_META 12
int ds3_hip_debug_grouped_lists(int32_t *meta, int32_t *counts, int32_t *offsets, int32_t *ids, float *wts,
                                int32_t *slot_pos, int32_t *tiles, int32_t *runs_gu, int32_t *runs_dn);

/* No ds3_metal.h counterpart (a test hook, like ds3_hip_debug_grouped_lists):
 * the run descriptors the grouped kernels start each run from, entry for
 * entry with that call's runs_gu / runs_dn (their counts are meta[5] and
 * meta[6] there): two int32 per run, { first list position of the run's work
 * item, expert << 16 | the work item's rows << 8 | n run }.  Synchronises;
 * -1 when no grouped call ran since the workspace last moved. */
int ds3_hip_debug_grouped_descs(int32_t *desc_gu, int32_t *desc_dn);

/* No ds3_metal.h counterpart: the row count of A from which
 * ds3_hip_matmul_quantized_batch takes its fp16 MFMA path (see there).  0
 * restores the default (64).  Returns the previous value. */
int ds3_hip_set_dense_mfma_min_rows(int min_rows);

/* ds3_hip_moe_ffn_batch uses the grouped (prefill) path when
 * n_tokens >= min_tokens, the per-token GEMV path otherwise.  0 restores the
 * default.  Returns the previous value. */
int ds3_hip_set_prefill_min_tokens(int min_tokens);

/* Per-kernel timing with HIP events on the library stream.  While enabled,
 * each kernel launch is bracketed by an event pair; ds3_hip_kernel_stats
 * synchronises and reports, for kernel i (0-based; returns -1 past the end),
 * its name, launch count and summed duration in milliseconds. */
void ds3_hip_kernel_timing(int enable);
/* Restrict kernel timing to launches of the kernel called `name` (NULL or ""
 * restores timing of every kernel), so that one kernel can be timed without
 * event pairs between the others. */
void ds3_hip_kernel_timing_only(const char *name);
void ds3_hip_kernel_timing_reset(void);
int  ds3_hip_kernel_stats(int i, char *name, size_t name_len, int64_t *count, double *total_ms);

/* Occupies the library stream for `us` microseconds (0 .. 1e6) with one
 * wave that touches no memory.  Enqueued ahead of kernels timed with
 * ds3_hip_kernel_timing when the host enqueues more slowly than the GPU runs
 * them (few tokens): the held stream lets the host queue the work first, so
 * that each event pair spans its kernel and not the host's enqueue.
 * Refused during graph capture. */
int ds3_hip_hold_stream(double us);

/* Event pair on the library stream around a caller-defined region. */
int    ds3_hip_timer_start(void);
double ds3_hip_timer_stop_ms(void);

/* Device name (e.g. "gfx950"), compute-unit count and HBM bytes. */
int ds3_hip_device_info(char *arch, size_t arch_len, int *n_cu, uint64_t *hbm_bytes);

/* HIP graphs (no ds3_metal.h counterpart; for callers that replay the same
 * calls many times, such as a decode step through every layer).  The calls
 * made between graph_begin and graph_end are captured on the library's
 * stream instead of run: they wait for nothing, nothing may be read back,
 * and the library's workspace must already be large enough (make the same
 * calls once before capturing; a call that would grow it fails).  The
 * captured calls hold no memset nodes.  graph_end returns an executable
 * graph; each graph_launch replays it on the library's stream with the
 * buffers the calls named (synchronous outside begin_batch / end_batch).
 * Not allowed while in batch mode or with kernel timing on.  During a capture
 * every entry point that would allocate, free, copy from or to the host or
 * wait (buffer_alloc / from_mmap / write / read, moe_ffn_experts,
 * synchronize, end_batch, router_stats, the timers, graph_launch) returns -1
 * (or does nothing) with a diagnostic; buffer_free is deferred to graph_end.
 * A live graph (graph_end .. graph_destroy) keeps the workspace block its
 * kernels address: a later eager call that needs a larger workspace gets a
 * new block and the old one is freed when the last live graph is destroyed.
 * Buffers the captured calls named must outlive the graph.  ds3_hip_shutdown
 * destroys every live graph. */
/* Test hook for the capture refusals above: marks a capture as open (on = 1)
 * or closed (0) without a device.  Refused (-1) once ds3_hip_init has run. */
int  ds3_hip_debug_simulate_capture(int on);
int  ds3_hip_graph_begin(void);
int  ds3_hip_graph_end(void **graph);
int  ds3_hip_graph_launch(void *graph);
void ds3_hip_graph_destroy(void *graph);

#ifdef __cplusplus
}
#endif

#endif /* DS3_HIP_H */
