/*
 * ds3_gen.h -- deterministic synthetic workloads for the MoE-FFN path.
 *
 * Counter-based random numbers (a splitmix64 finaliser over
 * (seed, stream, index)), Box-Muller normals, and GGUF block quantisers for
 * Q4_K / Q6_K / Q8_0 written from the block definitions the reference decodes
 * (reference src/ds3_reference.c:59-184).  The reference ships no usable
 * quantiser (its test helpers in tests/test_quant_utils.h:93-232 mis-pack
 * Q4_K nibbles and the second Q6_K half), so these are this project's own;
 * parity is defined on the quantised bytes, which GPU and oracle both decode.
 *
 * Every value depends only on (seed, stream, index): results do not depend on
 * the thread count or on how a matrix is split into calls.
 */
#ifndef DS3_GEN_H
#define DS3_GEN_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { DS3GEN_NORMAL = 0, DS3GEN_UNIFORM = 1 };

/* out[i] = value (offset + i) of the stream: NORMAL -> a + b * N(0,1),
 * UNIFORM -> U[a, b). */
void     ds3gen_fill(int dist, uint64_t seed, uint64_t stream, uint64_t offset,
                     int64_t n, double a, double b, float *out);

/* IEEE binary32 -> binary16, round to nearest even. */
uint16_t ds3gen_fp32_to_fp16(float f);

/* Quantise n floats (n a multiple of the block) into GGUF blocks.
 * type: 8 = Q8_0, 12 = Q4_K, 14 = Q6_K, 0 = F32 (copy).  Returns bytes
 * written or -1. */
int64_t  ds3gen_quantize(int type, const float *src, int64_t n, void *dst);

/* Bytes of one row of n_cols values of `type` (0 if unsupported). */
int64_t  ds3gen_row_bytes(int type, int64_t n_cols);

/* Generate a [n_rows][n_cols] matrix of `dist`(a, b) values from stream
 * `stream` (row-major element order) and quantise it row by row into dst
 * (n_rows * row_bytes).  Threads split rows.  Returns 0 / -1. */
int      ds3gen_matrix(int type, int dist, uint64_t seed, uint64_t stream,
                       int64_t n_rows, int64_t n_cols, double a, double b,
                       void *dst, int n_threads);

#ifdef __cplusplus
}
#endif

#endif /* DS3_GEN_H */
