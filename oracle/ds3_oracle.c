/*
 * ds3_oracle.c -- CPU restatement of the qw3 MoE-FFN path (test oracle).
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT: see ds3_oracle.h for who may load it and
 * what pins each function.  Citations are reference file:line.
 */
#include "ds3_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Scalars                                                                  */
/* ------------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, exact for every input
 * (src/ds3_reference.c:21-56).  Subnormal halves are m * 2^-24, which is a
 * normal float, so ldexpf is exact. */
float orc_fp16_to_fp32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15);
    const uint32_t expo = (uint32_t)(h >> 10) & 0x1fu;
    const uint32_t mant = (uint32_t)h & 0x3ffu;
    if (expo == 0) {
        float v = ldexpf((float)mant, -24);
        return sign ? -v : v;
    }
    uint32_t bits = sign << 31;
    if (expo == 0x1f)
        bits |= (0xffu << 23) | (mant << 13);           /* inf / nan */
    else
        bits |= ((expo + 112u) << 23) | (mant << 13);   /* rebias 15 -> 127 */
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------------------ */
/* Dequantisation                                                           */
/* ------------------------------------------------------------------------ */

/* 6-bit (scale, min) pair j of a Q4_K super-block's 12 packed scale bytes
 * (src/ds3_reference.c:76-85).  j < 4: low 6 bits of bytes j and j+4.
 * j >= 4: low / high nibble of byte j+4 plus the top 2 bits of bytes j-4 / j. */
static void q4k_scale_min(const uint8_t *s, int j, int *sc, int *mn)
{
    if (j < 4) {
        *sc = s[j] & 0x3f;
        *mn = s[j + 4] & 0x3f;
    } else {
        *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q4_K: 144-byte block {d f16, dmin f16, scales[12], qs[128]} -> 256 floats
 * (src/ds3_reference.c:87-113).  Weights 64g..64g+31 are the low nibbles of
 * qs[32g..32g+31] with sub-block 2g's (scale, min); weights 64g+32..64g+63
 * are the high nibbles with sub-block 2g+1's. */
static void deq_q4k_block(const uint8_t *b, float *y)
{
    const float d    = orc_fp16_to_fp32(rd16(b));
    const float dmin = orc_fp16_to_fp32(rd16(b + 2));
    const uint8_t *sc = b + 4;
    const uint8_t *qs = b + 16;
    for (int g = 0; g < 4; g++) {
        int s_lo, m_lo, s_hi, m_hi;
        q4k_scale_min(sc, 2 * g, &s_lo, &m_lo);
        q4k_scale_min(sc, 2 * g + 1, &s_hi, &m_hi);
        const float dl = d * (float)s_lo, ml = dmin * (float)m_lo;
        const float dh = d * (float)s_hi, mh = dmin * (float)m_hi;
        for (int l = 0; l < 32; l++) {
            const int q = qs[32 * g + l];
            y[64 * g + l]      = dl * (float)(q & 0x0f) - ml;
            y[64 * g + 32 + l] = dh * (float)(q >> 4) - mh;
        }
    }
}

/* Q6_K: 210-byte block {ql[128], qh[64], scales[16] int8, d f16 @208}
 * (src/ds3_reference.c:130-158).  Per 128-half h and l in 0..31 the four
 * 6-bit codes of outputs l, l+32, l+64, l+96 come from the low/high nibbles
 * of ql[64h+l], ql[64h+l+32] and the 2-bit fields of qh[32h+l]; output i
 * uses scale scales[i/16]. */
static void deq_q6k_block(const uint8_t *b, float *y)
{
    const float d = orc_fp16_to_fp32(rd16(b + 208));
    for (int h = 0; h < 2; h++) {
        const uint8_t *ql = b + 64 * h;
        const uint8_t *qh = b + 128 + 32 * h;
        const int8_t  *sc = (const int8_t *)(b + 192) + 8 * h;
        float *yh = y + 128 * h;
        for (int l = 0; l < 32; l++) {
            const int hb = qh[l];
            const int c0 = ((ql[l] & 0x0f)      | (((hb >> 0) & 3) << 4)) - 32;
            const int c1 = ((ql[l + 32] & 0x0f) | (((hb >> 2) & 3) << 4)) - 32;
            const int c2 = ((ql[l] >> 4)        | (((hb >> 4) & 3) << 4)) - 32;
            const int c3 = ((ql[l + 32] >> 4)   | (((hb >> 6) & 3) << 4)) - 32;
            const int is = l / 16;
            yh[l]      = d * (float)sc[is + 0] * (float)c0;
            yh[l + 32] = d * (float)sc[is + 2] * (float)c1;
            yh[l + 64] = d * (float)sc[is + 4] * (float)c2;
            yh[l + 96] = d * (float)sc[is + 6] * (float)c3;
        }
    }
}

/* Q8_0: 34-byte block {d f16, qs[32] int8} (src/ds3_reference.c:173-184). */
static void deq_q80_block(const uint8_t *b, float *y)
{
    const float d = orc_fp16_to_fp32(rd16(b));
    const int8_t *qs = (const int8_t *)(b + 2);
    for (int j = 0; j < 32; j++) y[j] = (float)qs[j] * d;
}

static int block_geom(int type, int *elems, int *bytes)
{
    switch (type) {
    case ORC_TYPE_F32:  *elems = 1;         *bytes = 4;             return 0;
    case ORC_TYPE_F16:  *elems = 1;         *bytes = 2;             return 0;
    case ORC_TYPE_Q8_0: *elems = ORC_QK8_0; *bytes = ORC_Q80_BYTES; return 0;
    case ORC_TYPE_Q4_K: *elems = ORC_QK_K;  *bytes = ORC_Q4K_BYTES; return 0;
    case ORC_TYPE_Q6_K: *elems = ORC_QK_K;  *bytes = ORC_Q6K_BYTES; return 0;
    default: return -1;
    }
}

size_t orc_row_bytes(int type, int64_t n_cols)
{
    int e, b;
    if (block_geom(type, &e, &b) != 0 || n_cols <= 0 || n_cols % e) return 0;
    return (size_t)(n_cols / e) * (size_t)b;
}

/* Decode n values (n a multiple of the block size) from raw bytes. */
static void deq_run(int type, const uint8_t *src, int64_t n, float *out)
{
    int64_t i;
    switch (type) {
    case ORC_TYPE_F32:
        memcpy(out, src, (size_t)n * sizeof(float));
        break;
    case ORC_TYPE_F16:
        for (i = 0; i < n; i++) out[i] = orc_fp16_to_fp32(rd16(src + 2 * i));
        break;
    case ORC_TYPE_Q8_0:
        for (i = 0; i < n / ORC_QK8_0; i++)
            deq_q80_block(src + i * ORC_Q80_BYTES, out + i * ORC_QK8_0);
        break;
    case ORC_TYPE_Q4_K:
        for (i = 0; i < n / ORC_QK_K; i++)
            deq_q4k_block(src + i * ORC_Q4K_BYTES, out + i * ORC_QK_K);
        break;
    case ORC_TYPE_Q6_K:
        for (i = 0; i < n / ORC_QK_K; i++)
            deq_q6k_block(src + i * ORC_Q6K_BYTES, out + i * ORC_QK_K);
        break;
    }
}

/* Whole-tensor dequantisation with the reference's checks
 * (src/ds3_reference.c:243-323): n > 0, n a multiple of the block size and
 * the buffer holding at least n/block blocks (F32/F16 are not size-checked
 * there either). */
int orc_dequantize(int type, const void *data, size_t size, int64_t n, float *out)
{
    int e, b;
    if (!data || !out || n <= 0 || block_geom(type, &e, &b) != 0) return -1;
    if (n % e) return -1;
    if (e > 1 && size < (size_t)(n / e) * (size_t)b) return -1;
    deq_run(type, (const uint8_t *)data, n, out);
    return 0;
}

/* One row, row stride nb1 bytes (src/ds3_reference.c:194-241). */
int orc_dequantize_row(int type, const void *data, uint64_t nb1,
                       int64_t n_rows, int64_t n_cols, int row, float *out)
{
    int e, b;
    if (!data || !out || row < 0 || row >= n_rows) return -1;
    if (block_geom(type, &e, &b) != 0 || n_cols % e) return -1;
    deq_run(type, (const uint8_t *)data + (size_t)row * nb1, n_cols, out);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Dense operators                                                          */
/* ------------------------------------------------------------------------ */

/* y[j] = sum_i x[i] * W[j][i], one float accumulator, i ascending
 * (src/ds3_reference.c:424-434). */
void orc_vec_matmul(const float *x, const float *W, float *y, int in_dim, int out_dim)
{
    for (int j = 0; j < out_dim; j++) {
        const float *row = W + (size_t)j * (size_t)in_dim;
        float acc = 0.0f;
        for (int i = 0; i < in_dim; i++) acc += x[i] * row[i];
        y[j] = acc;
    }
}

/* In-place softmax: subtract the max, expf, sequential sum, scale by the
 * reciprocal (src/ds3_reference.c:344-359). */
void orc_softmax(float *x, int n)
{
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float s = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        s += x[i];
    }
    const float r = 1.0f / s;
    for (int i = 0; i < n; i++) x[i] *= r;
}

/* k rounds of selection; a candidate must beat the running best strictly,
 * so equal scores resolve to the lowest index; the running best starts at
 * -1e30 (src/ds3_reference.c:466-490).  Returns -1 if a round finds nothing
 * (every remaining score <= -1e30 or NaN), where the reference would index
 * out of bounds. */
int orc_topk(const float *scores, int n, int k, int *idx, float *val)
{
    unsigned char *taken = (unsigned char *)calloc((size_t)n, 1);
    if (!taken) return -1;
    int rc = 0;
    for (int r = 0; r < k; r++) {
        int bi = -1;
        float bv = -1e30f;
        for (int j = 0; j < n; j++) {
            if (!taken[j] && scores[j] > bv) {
                bv = scores[j];
                bi = j;
            }
        }
        if (bi < 0) { rc = -1; break; }
        taken[bi] = 1;
        idx[r] = bi;
        val[r] = bv;
    }
    free(taken);
    return rc;
}

/* silu(x) = x / (1 + expf(-x)) (src/ds3_reference.c:436-441). */
void orc_silu(const float *x, float *out, int n)
{
    for (int i = 0; i < n; i++) out[i] = x[i] / (1.0f + expf(-x[i]));
}

void orc_mul(const float *a, const float *b, float *out, int n)
{
    for (int i = 0; i < n; i++) out[i] = a[i] * b[i];   /* src/ds3_reference.c:443-448 */
}

void orc_add(const float *a, const float *b, float *out, int n)
{
    for (int i = 0; i < n; i++) out[i] = a[i] + b[i];   /* src/ds3_reference.c:455-460 */
}

/* out = x * (1/sqrtf(mean(x^2) + eps)) * w (src/ds3_reference.c:329-342). */
void orc_rms_norm(const float *x, const float *w, float eps, int n, float *out)
{
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    ss /= (float)n;
    ss += eps;
    const float r = 1.0f / sqrtf(ss);
    for (int i = 0; i < n; i++) out[i] = x[i] * r * w[i];
}

/* ------------------------------------------------------------------------ */
/* MoE                                                                      */
/* ------------------------------------------------------------------------ */

/* softmax -> top-k -> renormalise by the reciprocal of the top-k sum when it
 * is positive (src/ds3_reference.c:628-639). */
void orc_route(float *logits, int n_expert, int n_used, bool norm_topk_prob,
               int *idx, float *scores)
{
    orc_softmax(logits, n_expert);
    orc_topk(logits, n_expert, n_used, idx, scores);
    if (norm_topk_prob) {
        float s = 0.0f;
        for (int i = 0; i < n_used; i++) s += scores[i];
        if (s > 0.0f) {
            const float r = 1.0f / s;
            for (int i = 0; i < n_used; i++) scores[i] *= r;
        }
    }
}

/* One expert's SwiGLU FFN on one token: h = silu(x.Wg) * (x.Wu), y = h.Wd
 * (src/ds3_reference.c:660-672).  g/u are [n_ff] scratch, y is [n_embd]. */
static void expert_ffn(const float *x, const float *wg, const float *wu,
                       const float *wd, float *g, float *u, float *y,
                       int n_embd, int n_ff)
{
    orc_vec_matmul(x, wg, g, n_embd, n_ff);
    orc_silu(g, g, n_ff);
    orc_vec_matmul(x, wu, u, n_embd, n_ff);
    orc_mul(g, u, g, n_ff);
    orc_vec_matmul(g, wd, y, n_ff, n_embd);
}

/* src/ds3_reference.c:605-710: router, softmax/top-k/renorm, then for each
 * selected expert in top-k order out[j] += w_i * y_i[j] starting from a zeroed
 * output, then the optional shared expert with weight 1. */
void orc_moe_ffn(const float *input, const float *w_gate_inp,
                 const float *w_gate_exps, const float *w_up_exps,
                 const float *w_down_exps,
                 const float *w_shared_gate, const float *w_shared_up,
                 const float *w_shared_down,
                 float *output, float *gate_logits, float *expert_scores,
                 int *expert_indices, int n_embd, int n_expert, int n_used,
                 int n_ff_exp, int n_ff_shared, bool norm_topk_prob)
{
    orc_vec_matmul(input, w_gate_inp, gate_logits, n_embd, n_expert);
    orc_route(gate_logits, n_expert, n_used, norm_topk_prob, expert_indices, expert_scores);

    memset(output, 0, (size_t)n_embd * sizeof(float));
    const int n_ff_max = n_ff_exp > n_ff_shared ? n_ff_exp : n_ff_shared;
    float *g = (float *)malloc((size_t)n_ff_max * sizeof(float));
    float *u = (float *)malloc((size_t)n_ff_max * sizeof(float));
    float *y = (float *)malloc((size_t)n_embd * sizeof(float));
    if (g && u && y) {
        const size_t per_gu = (size_t)n_ff_exp * (size_t)n_embd;
        for (int i = 0; i < n_used; i++) {
            const size_t e = (size_t)expert_indices[i];
            expert_ffn(input, w_gate_exps + e * per_gu, w_up_exps + e * per_gu,
                       w_down_exps + e * per_gu, g, u, y, n_embd, n_ff_exp);
            const float w = expert_scores[i];
            for (int j = 0; j < n_embd; j++) output[j] += w * y[j];
        }
        if (w_shared_gate && w_shared_up && w_shared_down) {
            expert_ffn(input, w_shared_gate, w_shared_up, w_shared_down,
                       g, u, y, n_embd, n_ff_shared);
            for (int j = 0; j < n_embd; j++) output[j] += y[j];
        }
    }
    free(g);
    free(u);
    free(y);
}

typedef struct {
    int T, tid, nth;
    const float *x, *wr, *wg, *wu, *wd;
    float *out, *logits, *scores;
    int *idx;
    int n_embd, n_expert, n_used, n_ff;
    bool norm;
} tok_job_t;

static void *tok_worker(void *arg)
{
    const tok_job_t *j = (const tok_job_t *)arg;
    for (int t = j->tid; t < j->T; t += j->nth) {
        orc_moe_ffn(j->x + (size_t)t * j->n_embd, j->wr, j->wg, j->wu, j->wd,
                    NULL, NULL, NULL,
                    j->out + (size_t)t * j->n_embd,
                    j->logits + (size_t)t * j->n_expert,
                    j->scores + (size_t)t * j->n_used,
                    j->idx + (size_t)t * j->n_used,
                    j->n_embd, j->n_expert, j->n_used, j->n_ff, 0, j->norm);
    }
    return NULL;
}

int orc_moe_ffn_tokens(int T, const float *x, const float *w_gate_inp,
                       const float *w_gate_exps, const float *w_up_exps,
                       const float *w_down_exps, float *out, float *logits,
                       float *scores, int *idx, int n_embd, int n_expert,
                       int n_used, int n_ff_exp, bool norm_topk_prob,
                       int n_threads)
{
    if (T <= 0) return 0;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > T) n_threads = T;
    if (n_threads > 256) n_threads = 256;
    pthread_t th[256];
    unsigned char spawned[256] = { 0 };
    tok_job_t jobs[256];
    for (int i = 0; i < n_threads; i++) {
        jobs[i] = (tok_job_t){ T, i, n_threads, x, w_gate_inp, w_gate_exps, w_up_exps,
                               w_down_exps, out, logits, scores, idx,
                               n_embd, n_expert, n_used, n_ff_exp, norm_topk_prob };
    }
    /* shares 1..n-1 on threads; share 0 (and any share that fails to spawn)
     * runs on the calling thread */
    for (int i = 1; i < n_threads; i++)
        spawned[i] = pthread_create(&th[i], NULL, tok_worker, &jobs[i]) == 0;
    tok_worker(&jobs[0]);
    for (int i = 1; i < n_threads; i++) {
        if (spawned[i]) pthread_join(th[i], NULL);
        else tok_worker(&jobs[i]);
    }
    return 0;
}

/* Bucketing in token order (src/ds3_engine.c:932-955), compacted by an
 * exclusive prefix over the per-expert counts. */
int orc_bucket(int T, int n_used, int n_expert, const int *idx, const float *scores,
               int *counts, int *offsets, int *ids, float *wts, int *slot_pos)
{
    for (int e = 0; e < n_expert; e++) counts[e] = 0;
    for (int s = 0; s < T * n_used; s++) {
        const int e = idx[s];
        if (e < 0 || e >= n_expert) return -1;
        counts[e]++;
    }
    int run = 0;
    for (int e = 0; e < n_expert; e++) {
        offsets[e] = run;
        run += counts[e];
    }
    int *fill = (int *)calloc((size_t)n_expert, sizeof(int));
    if (!fill) return -1;
    for (int t = 0; t < T; t++) {
        for (int k = 0; k < n_used; k++) {
            const int e = idx[t * n_used + k];
            const int p = offsets[e] + fill[e]++;
            ids[p] = t;
            wts[p] = scores[t * n_used + k];
            if (slot_pos) slot_pos[t * n_used + k] = p;
        }
    }
    free(fill);
    return 0;
}

/* src/ds3_engine.c:895-1022 without the shared expert: zero the output,
 * bucket, then per expert 0..n_expert-1 with tokens: gather rows, gate and
 * up products, silu(g)*u, down product, out[token] += w * y in list order. */
int orc_moe_gathered(int T, const float *x, const int *idx, const float *scores,
                     const float *w_gate_exps, const float *w_up_exps,
                     const float *w_down_exps, float *out,
                     int n_embd, int n_expert, int n_used, int n_ff_exp)
{
    const int S = T * n_used;
    int *counts  = (int *)malloc((size_t)n_expert * sizeof(int));
    int *offsets = (int *)malloc((size_t)n_expert * sizeof(int));
    int *ids     = (int *)malloc((size_t)(S > 0 ? S : 1) * sizeof(int));
    float *wts   = (float *)malloc((size_t)(S > 0 ? S : 1) * sizeof(float));
    float *g = (float *)malloc((size_t)n_ff_exp * sizeof(float));
    float *u = (float *)malloc((size_t)n_ff_exp * sizeof(float));
    float *y = (float *)malloc((size_t)n_embd * sizeof(float));
    int rc = -1;
    if (!counts || !offsets || !ids || !wts || !g || !u || !y) goto done;
    memset(out, 0, (size_t)T * (size_t)n_embd * sizeof(float));
    if (orc_bucket(T, n_used, n_expert, idx, scores, counts, offsets, ids, wts, NULL) != 0)
        goto done;
    const size_t per = (size_t)n_ff_exp * (size_t)n_embd;
    for (int e = 0; e < n_expert; e++) {
        for (int c = 0; c < counts[e]; c++) {
            const int p = offsets[e] + c;
            const float *xr = x + (size_t)ids[p] * n_embd;
            expert_ffn(xr, w_gate_exps + e * per, w_up_exps + e * per,
                       w_down_exps + e * per, g, u, y, n_embd, n_ff_exp);
            float *o = out + (size_t)ids[p] * n_embd;
            for (int j = 0; j < n_embd; j++) o[j] += wts[p] * y[j];
        }
    }
    rc = 0;
done:
    free(counts); free(offsets); free(ids); free(wts);
    free(g); free(u); free(y);
    return rc;
}
