/*
 * ds3_oracle.h -- CPU restatement of the qw3 MoE-FFN path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker.
 * The product (qw3_amd / libds3_hip.so) never links or calls it.
 *
 * Every function restates one piece of the reference's algorithm and names
 * the reference file:line it follows (paths relative to the reference root).
 * Build flags: -O2 -ffp-contract=off, no -march=native, so float arithmetic
 * rounds exactly like the reference's baseline x86-64 build (no FMA).
 *
 * Pinning (what checks each function, beyond retyping it):
 *   dequant (Q4_K/Q6_K/Q8_0/F16/F32): the reference's own KATs
 *     (tests/test_reference.c:215-418) as JSON fixtures, closed-form exactness
 *     (every dequantised value is an exact product, one rounding for Q4_K),
 *     and byte-for-byte equality against the compiled reference (oracle/_ref).
 *   vec_matmul / softmax / topk / silu / rms_norm / add: reference KATs
 *     (test_reference.c:32-178) + bit-exact equality against oracle/_ref +
 *     brute force / invariants on tiny inputs.
 *   moe_ffn: bit-exact against oracle/_ref ds3_ref_moe_ffn on seeded inputs.
 *   bucket / moe_gathered: invariants (sum of counts = T*k, token order per
 *     expert, round trip of (token, slot) ids) and agreement of the gathered
 *     output with per-token moe_ffn within float tolerance.
 */
#ifndef DS3_ORACLE_H
#define DS3_ORACLE_H

#include <stdint.h>
#include <stddef.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids used on this path (reference src/ds3.h:201-216). */
enum {
    ORC_TYPE_F32  = 0,
    ORC_TYPE_F16  = 1,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q6_K = 14,
};

/* Block geometry (reference src/ds3_reference.c:62-74, 119-128, 164-171). */
#define ORC_QK_K        256
#define ORC_Q4K_BYTES   144
#define ORC_Q6K_BYTES   210
#define ORC_QK8_0       32
#define ORC_Q80_BYTES   34

float   orc_fp16_to_fp32(uint16_t h);

/* Bytes a [n_rows][n_cols] matrix of `type` occupies (0 if n_cols does not
 * fit the block size). */
size_t  orc_row_bytes(int type, int64_t n_cols);

/* Dequantise n contiguous values (n a multiple of the block size).
 * Mirrors ds3_ref_dequantize_tensor (src/ds3_reference.c:243-323):
 * returns -1 on bad type / n not a block multiple / size < needed. */
int     orc_dequantize(int type, const void *data, size_t size, int64_t n, float *out);

/* One row of a [n_rows][n_cols] tensor with byte row stride nb1
 * (src/ds3_reference.c:194-241). */
int     orc_dequantize_row(int type, const void *data, uint64_t nb1,
                           int64_t n_rows, int64_t n_cols, int row, float *out);

void    orc_vec_matmul(const float *x, const float *W, float *y, int in_dim, int out_dim);
void    orc_softmax(float *x, int n);
int     orc_topk(const float *scores, int n, int k, int *idx, float *val);
void    orc_silu(const float *x, float *out, int n);
void    orc_mul(const float *a, const float *b, float *out, int n);
void    orc_add(const float *a, const float *b, float *out, int n);
void    orc_rms_norm(const float *x, const float *w, float eps, int n, float *out);

/* Router stage alone: logits -> softmax -> top-k -> renorm
 * (src/ds3_reference.c:627-639).  `logits` is overwritten by the probs. */
void    orc_route(float *logits, int n_expert, int n_used, bool norm_topk_prob,
                  int *idx, float *scores);

/* One token of the MoE FFN (src/ds3_reference.c:605-710).  Weights are FP32,
 * expert-major: gate/up [n_expert][n_ff][n_embd], down [n_expert][n_embd][n_ff].
 * Shared-expert pointers may be NULL. */
void    orc_moe_ffn(const float *input, const float *w_gate_inp,
                    const float *w_gate_exps, const float *w_up_exps,
                    const float *w_down_exps,
                    const float *w_shared_gate, const float *w_shared_up,
                    const float *w_shared_down,
                    float *output, float *gate_logits, float *expert_scores,
                    int *expert_indices, int n_embd, int n_expert, int n_used,
                    int n_ff_exp, int n_ff_shared, bool norm_topk_prob);

/* T independent tokens of orc_moe_ffn on n_threads pthreads (the function is
 * reentrant).  x [T][n_embd] -> out [T][n_embd], idx/scores [T][n_used],
 * logits [T][n_expert] (softmax probs after the call, as in the reference). */
int     orc_moe_ffn_tokens(int T, const float *x, const float *w_gate_inp,
                           const float *w_gate_exps, const float *w_up_exps,
                           const float *w_down_exps, float *out, float *logits,
                           float *scores, int *idx, int n_embd, int n_expert,
                           int n_used, int n_ff_exp, bool norm_topk_prob,
                           int n_threads);

/* Token->expert bucketing of the gathered prefill path
 * (src/ds3_engine.c:932-955): for each token t in order and each slot k,
 * append t to expert idx[t][k]'s list.  Outputs are compacted:
 *   counts[e], offsets[e] (exclusive prefix of counts),
 *   ids[offsets[e] + c] = token, wts[offsets[e] + c] = its routing weight,
 *   slot_pos[t*n_used + k] = offsets[e] + c  (where that slot landed).
 * Returns -1 on an out-of-range expert id. */
int     orc_bucket(int T, int n_used, int n_expert, const int *idx, const float *scores,
                   int *counts, int *offsets, int *ids, float *wts, int *slot_pos);

/* Gathered prefill MoE (src/ds3_engine.c:895-1022): bucket, then for each
 * expert in order 0..n_expert-1 gather its rows, gate/up/down, SwiGLU, and
 * scatter-add w * y into out (expert order, as the engine accumulates).
 * `out` [T][n_embd] is zeroed first (src/ds3_engine.c:902).  Routing comes
 * from idx/scores [T][n_used] (the caller runs orc_route per token). */
int     orc_moe_gathered(int T, const float *x, const int *idx, const float *scores,
                         const float *w_gate_exps, const float *w_up_exps,
                         const float *w_down_exps, float *out,
                         int n_embd, int n_expert, int n_used, int n_ff_exp);

#ifdef __cplusplus
}
#endif

#endif /* DS3_ORACLE_H */
