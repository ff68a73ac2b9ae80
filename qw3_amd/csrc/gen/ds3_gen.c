/*
 * ds3_gen.c -- deterministic synthetic workloads and GGUF block quantisers.
 * See ds3_gen.h.  Block layouts follow the decoders in the reference
 * (src/ds3_reference.c:59-184); the quantisation rules are this project's.
 */
#include "ds3_gen.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Random numbers                                                           */
/* ------------------------------------------------------------------------ */

static inline uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t stream_key(uint64_t seed, uint64_t stream)
{
    return mix64(seed ^ mix64(stream * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull));
}

static inline double unit_open0(uint64_t h) { return ((double)(h >> 11) + 1.0) * 0x1.0p-53; }
static inline double unit_closed0(uint64_t h) { return (double)(h >> 11) * 0x1.0p-53; }

void ds3gen_fill(int dist, uint64_t seed, uint64_t stream, uint64_t offset,
                 int64_t n, double a, double b, float *out)
{
    const uint64_t key = stream_key(seed, stream);
    for (int64_t i = 0; i < n; i++) {
        const uint64_t c = offset + (uint64_t)i;
        const uint64_t h1 = mix64(key + 2 * c);
        if (dist == DS3GEN_UNIFORM) {
            out[i] = (float)(a + (b - a) * unit_closed0(h1));
        } else {
            const uint64_t h2 = mix64(key + 2 * c + 1);
            const double r = sqrt(-2.0 * log(unit_open0(h1)));
            const double z = r * cos(6.283185307179586476925 * unit_closed0(h2));
            out[i] = (float)(a + b * z);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Half precision                                                           */
/* ------------------------------------------------------------------------ */

uint16_t ds3gen_fp32_to_fp16(float f)
{
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u)                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u)                       /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {                      /* below 2^-14: half subnormal */
        float af;
        memcpy(&af, &ax, sizeof af);
        return (uint16_t)(sign | (uint32_t)rintf(af * 16777216.0f));
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float fp16_value(uint16_t h)
{
    const uint32_t s = h >> 15, e = (h >> 10) & 31u, m = h & 1023u;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024u), (int)e - 25);
    return s ? -v : v;
}

static void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

static int clampi(long v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : (int)v); }

/* ------------------------------------------------------------------------ */
/* Block quantisers                                                         */
/* ------------------------------------------------------------------------ */

/* Q8_0: d = max|x| / 127 (stored f16), q = round(x / d). */
static void quant_q80(const float *x, uint8_t *b)
{
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    const uint16_t d16 = ds3gen_fp32_to_fp16(amax / 127.0f);
    const float d = fp16_value(d16);
    put16(b, d16);
    for (int i = 0; i < 32; i++)
        b[2 + i] = (uint8_t)(int8_t)(d > 0.0f ? clampi(lrintf(x[i] / d), -128, 127) : 0);
}

/* Q4_K: each 32-value sub-block j is x ~= S_j * q - M_j, q in 0..15, with
 * S_j = d * sc_j and M_j = dmin * m_j, sc_j / m_j 6-bit, d / dmin f16. */
static void quant_q4k(const float *x, uint8_t *b)
{
    float s[8], m[8], smax = 0.0f, mmax = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int i = 0; i < 32; i++) {
            lo = fminf(lo, x[32 * j + i]);
            hi = fmaxf(hi, x[32 * j + i]);
        }
        s[j] = (hi - lo) / 15.0f;
        m[j] = -lo;
        smax = fmaxf(smax, s[j]);
        mmax = fmaxf(mmax, m[j]);
    }
    const uint16_t d16 = ds3gen_fp32_to_fp16(smax / 63.0f);
    const uint16_t m16 = ds3gen_fp32_to_fp16(mmax / 63.0f);
    const float d = fp16_value(d16), dmin = fp16_value(m16);
    int sc[8], mq[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0.0f ? clampi(lrintf(s[j] / d), 0, 63) : 0;
        mq[j] = dmin > 0.0f ? clampi(lrintf(m[j] / dmin), 0, 63) : 0;
    }
    put16(b, d16);
    put16(b + 2, m16);
    uint8_t *ps = b + 4;
    for (int j = 0; j < 4; j++) {
        ps[j]     = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        ps[j + 4] = (uint8_t)((mq[j] & 63) | ((mq[j + 4] >> 4) << 6));
        ps[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mq[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        const float S = d * (float)sc[j], M = dmin * (float)mq[j];
        for (int i = 0; i < 32; i++)
            q[32 * j + i] = (uint8_t)(S > 0.0f ? clampi(lrintf((x[32 * j + i] + M) / S), 0, 15) : 0);
    }
    uint8_t *qs = b + 16;
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++)
            qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
}

/* Q6_K: each 16-value group g is x ~= d * sc_g * (c - 32), c in 0..63,
 * sc_g int8, d f16; codes packed 4+2 bits as the decoder expects. */
static void quant_q6k(const float *x, uint8_t *b)
{
    float s[16], smax = 0.0f;
    for (int g = 0; g < 16; g++) {
        float amax = 0.0f;
        for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(x[16 * g + i]));
        s[g] = amax / 31.0f;
        smax = fmaxf(smax, s[g]);
    }
    const uint16_t d16 = ds3gen_fp32_to_fp16(smax / 127.0f);
    const float d = fp16_value(d16);
    int8_t sc[16];
    uint8_t c[256];
    for (int g = 0; g < 16; g++) {
        sc[g] = (int8_t)(d > 0.0f ? clampi(lrintf(s[g] / d), -128, 127) : 0);
        const float S = d * (float)sc[g];
        for (int i = 0; i < 16; i++)
            c[16 * g + i] = (uint8_t)((S != 0.0f ? clampi(lrintf(x[16 * g + i] / S), -32, 31) : 0) + 32);
    }
    for (int h = 0; h < 2; h++) {
        uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
        const uint8_t *ch = c + 128 * h;
        for (int l = 0; l < 32; l++) {
            const int c0 = ch[l], c1 = ch[l + 32], c2 = ch[l + 64], c3 = ch[l + 96];
            ql[l]      = (uint8_t)((c0 & 15) | ((c2 & 15) << 4));
            ql[l + 32] = (uint8_t)((c1 & 15) | ((c3 & 15) << 4));
            qh[l]      = (uint8_t)((c0 >> 4) | ((c1 >> 4) << 2) | ((c2 >> 4) << 4) | ((c3 >> 4) << 6));
        }
    }
    memcpy(b + 192, sc, 16);
    put16(b + 208, d16);
}

int64_t ds3gen_row_bytes(int type, int64_t n_cols)
{
    switch (type) {
    case 0:  return n_cols * 4;
    case 8:  return n_cols % 32  ? 0 : n_cols / 32 * 34;
    case 12: return n_cols % 256 ? 0 : n_cols / 256 * 144;
    case 14: return n_cols % 256 ? 0 : n_cols / 256 * 210;
    default: return 0;
    }
}

int64_t ds3gen_quantize(int type, const float *src, int64_t n, void *dst)
{
    const int64_t nbytes = ds3gen_row_bytes(type, n);
    if (n <= 0 || nbytes <= 0) return -1;
    uint8_t *o = (uint8_t *)dst;
    int64_t i;
    switch (type) {
    case 0:  memcpy(dst, src, (size_t)n * 4); break;
    case 8:  for (i = 0; i < n / 32; i++)  quant_q80(src + 32 * i, o + 34 * i);  break;
    case 12: for (i = 0; i < n / 256; i++) quant_q4k(src + 256 * i, o + 144 * i); break;
    case 14: for (i = 0; i < n / 256; i++) quant_q6k(src + 256 * i, o + 210 * i); break;
    }
    return nbytes;
}

/* ------------------------------------------------------------------------ */
/* Matrices                                                                 */
/* ------------------------------------------------------------------------ */

typedef struct {
    int type, dist;
    uint64_t seed, stream;
    int64_t r0, r1, n_cols, row_bytes;
    double a, b;
    uint8_t *dst;
    int rc;
} mat_job_t;

static void *mat_worker(void *p)
{
    mat_job_t *j = (mat_job_t *)p;
    float *tmp = (float *)malloc((size_t)j->n_cols * sizeof(float));
    if (!tmp) { j->rc = -1; return NULL; }
    for (int64_t r = j->r0; r < j->r1; r++) {
        ds3gen_fill(j->dist, j->seed, j->stream, (uint64_t)r * (uint64_t)j->n_cols,
                    j->n_cols, j->a, j->b, tmp);
        ds3gen_quantize(j->type, tmp, j->n_cols, j->dst + r * j->row_bytes);
    }
    free(tmp);
    j->rc = 0;
    return NULL;
}

int ds3gen_matrix(int type, int dist, uint64_t seed, uint64_t stream,
                  int64_t n_rows, int64_t n_cols, double a, double b,
                  void *dst, int n_threads)
{
    const int64_t rb = ds3gen_row_bytes(type, n_cols);
    if (rb <= 0 || n_rows <= 0 || !dst) return -1;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    if (n_threads > n_rows) n_threads = (int)n_rows;
    pthread_t th[64];
    unsigned char spawned[64] = { 0 };
    mat_job_t jobs[64];
    for (int i = 0; i < n_threads; i++) {
        jobs[i] = (mat_job_t){ type, dist, seed, stream,
                               n_rows * i / n_threads, n_rows * (i + 1) / n_threads,
                               n_cols, rb, a, b, (uint8_t *)dst, -1 };
    }
    for (int i = 1; i < n_threads; i++)
        spawned[i] = pthread_create(&th[i], NULL, mat_worker, &jobs[i]) == 0;
    mat_worker(&jobs[0]);
    int rc = jobs[0].rc;
    for (int i = 1; i < n_threads; i++) {
        if (spawned[i]) pthread_join(th[i], NULL);
        else mat_worker(&jobs[i]);
        if (jobs[i].rc != 0) rc = -1;
    }
    return rc;
}
