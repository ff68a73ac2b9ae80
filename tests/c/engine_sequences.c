/*
 * engine_sequences.c -- the reference engine's MoE call sequences, replayed
 * through the ds3_metal_* names of include/ds3_metal_compat.h against
 * libds3_hip.so.  Test harness: tests/test_gpu_engine.py writes the inputs and
 * checks the outputs against the CPU oracle.
 *
 * Weights come the way the engine gets them from a GGUF file: one page-aligned
 * mapping imported with ds3_metal_buffer_from_mmap (reference
 * src/ds3_metal.m:387-414), each tensor a view at its data offset.
 *
 *   decode  (reference src/ds3_engine.c:519-597, 1425-1450): per token
 *           rms_norm -> zero ffn_out -> moe_ffn_router -> begin_batch,
 *           moe_router_topk_batch, end_batch -> read indices/scores ->
 *           moe_ffn_experts (host indices) -> vec_add(ffn_out, residual)
 *   prefill (reference src/ds3_engine.c:860-893, 895-1022, 1137-1150):
 *           rms_norm of M rows -> moe_ffn_router per token into a logits
 *           row -> moe_router_topk_batch_tokens -> read back -> host
 *           bucketing -> per expert gather_rows, matmul_quantized_batch
 *           x3, silu_mul, scatter_add_weighted -> vec_add(ffn_out, residual)
 *
 * and the device-routed sequences that replace the host read-back and host
 * bucketing on a discrete GPU (no ds3_metal.h counterpart for the last three):
 *   gpu-only decode (reference src/ds3_engine.c:638-720): per token rms_norm
 *           -> zero ffn_out -> moe_ffn (router, top-k and experts on the
 *           device, expert offset table) -> vec_add(ffn_out, residual)
 *   block   per token ds3_hip_moe_block: hidden += MoE(rms_norm(hidden) * g)
 *           in place, the engine's whole FFN block in one call
 *   graph   the same T block calls captured once as a HIP graph
 *           (ds3_hip_graph_begin / _end) and replayed on the same input
 *   batch   the prefill chunk in one ds3_hip_moe_ffn_batch call (routing,
 *           bucketing, grouped products and combine on the device) into the
 *           zeroed ffn_out, with the residual added by the call
 *
 * Usage: engine_sequences <dir>, with <dir>/meta.txt holding
 *   E K F k T gate_type up_type down_type off_router off_gate off_up off_down
 *   blob_bytes
 * and <dir>/{weights.bin, hidden.f32, gain.f32, residual.f32}.  Writes
 * <dir>/{decode_out.f32, decode_idx.i32, prefill_out.f32, prefill_idx.i32,
 * norm.f32, gpuonly_out.f32, block_out.f32, block_idx.i32, graph_out.f32,
 * batch_out.f32, batch_idx.i32}.  Exit status 0 on success.
 */
#define _DEFAULT_SOURCE
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "ds3_metal_compat.h"

#define CHECK(x)                                                                     \
    do {                                                                             \
        if (!(x)) {                                                                  \
            fprintf(stderr, "engine_sequences: FAIL %s at line %d\n", #x, __LINE__); \
            return 1;                                                                \
        }                                                                            \
    } while (0)

static const float NORM_EPS = 1e-6f;

static size_t row_bytes(int type, uint32_t n)
{
    switch (type) {
    case DS3_HIP_TYPE_F32: return (size_t)n * 4;
    case DS3_HIP_TYPE_Q8_0: return (size_t)n / 32 * 34;
    case DS3_HIP_TYPE_Q4_K: return (size_t)n / 256 * 144;
    case DS3_HIP_TYPE_Q6_K: return (size_t)n / 256 * 210;
    default: return 0;
    }
}

static void *read_file(const char *dir, const char *name, size_t bytes)
{
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    void *p = malloc(bytes);
    if (p && fread(p, 1, bytes, f) != bytes) {
        free(p);
        p = NULL;
    }
    fclose(f);
    return p;
}

static int write_file(const char *dir, const char *name, const void *p, size_t bytes)
{
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f) return -1;
    const size_t w = fwrite(p, 1, bytes, f);
    fclose(f);
    return w == bytes ? 0 : -1;
}

int main(int argc, char **argv)
{
    if (argc != 2) {
        fprintf(stderr, "usage: engine_sequences <dir>\n");
        return 2;
    }
    const char *dir = argv[1];
    char path[4096];
    snprintf(path, sizeof path, "%s/meta.txt", dir);
    FILE *mf = fopen(path, "r");
    CHECK(mf != NULL);
    unsigned E, K, F, k, T;
    int gt, ut, dt;
    unsigned long long off_r, off_g, off_u, off_d, blob;
    const int nread = fscanf(mf, "%u %u %u %u %u %d %d %d %llu %llu %llu %llu %llu", &E, &K, &F, &k, &T, &gt, &ut,
                             &dt, &off_r, &off_g, &off_u, &off_d, &blob);
    fclose(mf);
    CHECK(nread == 13);
    const size_t gs = row_bytes(gt, K), us = row_bytes(ut, K), ds = row_bytes(dt, F), rs = row_bytes(0, K);

    CHECK(ds3_metal_init() == 0);

    /* the GGUF tensor data: one read-only mapping, imported whole */
    snprintf(path, sizeof path, "%s/weights.bin", dir);
    const int fd = open(path, O_RDONLY);
    CHECK(fd >= 0);
    void *map = mmap(NULL, blob, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    CHECK(map != MAP_FAILED);
    ds3_metal_buffer_t *wbuf = ds3_metal_buffer_from_mmap(map, blob);
    CHECK(wbuf != NULL);
    const unsigned char probe = 0;
    CHECK(ds3_metal_buffer_write(wbuf, 0, &probe, 1) != 0);    /* imported weights refuse writes */
    ds3_metal_buffer_t *router = ds3_metal_buffer_view(wbuf, off_r, (size_t)E * rs);
    ds3_metal_buffer_t *gate = ds3_metal_buffer_view(wbuf, off_g, (size_t)E * F * gs);
    ds3_metal_buffer_t *up = ds3_metal_buffer_view(wbuf, off_u, (size_t)E * F * us);
    ds3_metal_buffer_t *down = ds3_metal_buffer_view(wbuf, off_d, (size_t)E * K * ds);
    CHECK(router && gate && up && down);

    float *hidden = read_file(dir, "hidden.f32", (size_t)T * K * 4);
    float *gain = read_file(dir, "gain.f32", (size_t)K * 4);
    float *residual = read_file(dir, "residual.f32", (size_t)T * K * 4);
    CHECK(hidden && gain && residual);
    float *out = malloc((size_t)T * K * 4), *norm_rows = malloc((size_t)T * K * 4);
    int32_t *idx_all = malloc((size_t)T * k * 4);
    float *sc_all = malloc((size_t)T * k * 4);
    CHECK(out && norm_rows && idx_all && sc_all);

    ds3_metal_buffer_t *b_ffn_norm = ds3_metal_buffer_alloc((size_t)K * 4);
    CHECK(b_ffn_norm && ds3_metal_buffer_write(b_ffn_norm, 0, gain, (size_t)K * 4) == 0);

    /* ---------------------------------------------------------------- decode */
    {
        ds3_metal_buffer_t *b_hidden = ds3_metal_buffer_alloc((size_t)K * 4);
        ds3_metal_buffer_t *b_norm = ds3_metal_buffer_alloc((size_t)K * 4);
        ds3_metal_buffer_t *b_res = ds3_metal_buffer_alloc((size_t)K * 4);
        ds3_metal_buffer_t *b_ffn = ds3_metal_buffer_alloc((size_t)K * 4);
        ds3_metal_buffer_t *b_logits = ds3_metal_buffer_alloc((size_t)E * 4);
        ds3_metal_buffer_t *b_idx = ds3_metal_buffer_alloc((size_t)k * 4);
        ds3_metal_buffer_t *b_sc = ds3_metal_buffer_alloc((size_t)k * 4);
        ds3_metal_buffer_t *b_mh = ds3_metal_buffer_alloc((size_t)k * F * 4);
        ds3_metal_buffer_t *b_mu = ds3_metal_buffer_alloc((size_t)k * F * 4);
        ds3_metal_buffer_t *b_md = ds3_metal_buffer_alloc((size_t)k * K * 4);
        CHECK(b_hidden && b_norm && b_res && b_ffn && b_logits && b_idx && b_sc && b_mh && b_mu && b_md);
        for (unsigned t = 0; t < T; t++) {
            CHECK(ds3_metal_buffer_write(b_hidden, 0, hidden + (size_t)t * K, (size_t)K * 4) == 0);
            CHECK(ds3_metal_buffer_write(b_res, 0, residual + (size_t)t * K, (size_t)K * 4) == 0);
            CHECK(ds3_metal_rms_norm(b_hidden, b_ffn_norm, b_norm, K, 1, NORM_EPS) == 0);
            CHECK(ds3_metal_buffer_zero_f32(b_ffn, (size_t)K * 4) == 0);
            CHECK(ds3_metal_moe_ffn_router(b_norm, router, b_logits, K, E, rs, DS3_HIP_TYPE_F32) == 0);
            CHECK(ds3_metal_begin_batch() == 0);
            CHECK(ds3_metal_moe_router_topk_batch(b_logits, b_idx, b_sc, 1, E, k, true) == 0);
            ds3_metal_end_batch();
            int32_t idx_h[16];
            float sc_h[16];
            CHECK(ds3_metal_buffer_read(b_idx, 0, idx_h, (size_t)k * 4) == 0);
            CHECK(ds3_metal_buffer_read(b_sc, 0, sc_h, (size_t)k * 4) == 0);
            CHECK(ds3_metal_moe_ffn_experts(b_norm, gate, up, down, gt, ut, dt, gs, us, ds, NULL, NULL, NULL,
                                            DS3_HIP_TYPE_F32, DS3_HIP_TYPE_F32, DS3_HIP_TYPE_F32, 0, 0, 0, b_ffn, b_mh,
                                            b_mu, b_md, K, k, F, 0, idx_h, sc_h) == 0);
            CHECK(ds3_metal_vec_add(b_ffn, b_res, b_hidden, K) == 0);
            CHECK(ds3_metal_buffer_read(b_hidden, 0, out + (size_t)t * K, (size_t)K * 4) == 0);
            CHECK(ds3_metal_buffer_read(b_norm, 0, norm_rows + (size_t)t * K, (size_t)K * 4) == 0);
            memcpy(idx_all + (size_t)t * k, idx_h, (size_t)k * 4);
        }
        CHECK(write_file(dir, "decode_out.f32", out, (size_t)T * K * 4) == 0);
        CHECK(write_file(dir, "decode_idx.i32", idx_all, (size_t)T * k * 4) == 0);
        CHECK(write_file(dir, "norm.f32", norm_rows, (size_t)T * K * 4) == 0);
        ds3_metal_buffer_t *bs[] = { b_hidden, b_norm, b_res, b_ffn, b_logits, b_idx, b_sc, b_mh, b_mu, b_md };
        for (size_t i = 0; i < sizeof bs / sizeof bs[0]; i++) ds3_metal_buffer_free(bs[i]);
    }

    /* --------------------------------------------------------------- prefill */
    {
        const unsigned M = T;
        ds3_metal_buffer_t *b_hidden = ds3_metal_buffer_alloc((size_t)M * K * 4);
        ds3_metal_buffer_t *b_norm = ds3_metal_buffer_alloc((size_t)M * K * 4);
        ds3_metal_buffer_t *b_res = ds3_metal_buffer_alloc((size_t)M * K * 4);
        ds3_metal_buffer_t *b_ffn = ds3_metal_buffer_alloc((size_t)M * K * 4);
        ds3_metal_buffer_t *b_logits = ds3_metal_buffer_alloc((size_t)M * E * 4);
        ds3_metal_buffer_t *b_idx = ds3_metal_buffer_alloc((size_t)M * k * 4);
        ds3_metal_buffer_t *b_sc = ds3_metal_buffer_alloc((size_t)M * k * 4);
        ds3_metal_buffer_t *b_gids = ds3_metal_buffer_alloc((size_t)E * M * 4);
        ds3_metal_buffer_t *b_gsc = ds3_metal_buffer_alloc((size_t)E * M * 4);
        ds3_metal_buffer_t *b_mh = ds3_metal_buffer_alloc((size_t)M * F * 4);
        ds3_metal_buffer_t *b_mu = ds3_metal_buffer_alloc((size_t)M * F * 4);
        ds3_metal_buffer_t *b_md = ds3_metal_buffer_alloc((size_t)M * K * 4);
        CHECK(b_hidden && b_norm && b_res && b_ffn && b_logits && b_idx && b_sc && b_gids && b_gsc && b_mh && b_mu &&
              b_md);
        CHECK(ds3_metal_buffer_write(b_hidden, 0, hidden, (size_t)M * K * 4) == 0);
        CHECK(ds3_metal_buffer_write(b_res, 0, residual, (size_t)M * K * 4) == 0);
        CHECK(ds3_metal_rms_norm(b_hidden, b_ffn_norm, b_norm, K, M, NORM_EPS) == 0);
        for (unsigned t = 0; t < M; t++) {
            ds3_metal_buffer_t *nv = ds3_metal_buffer_view(b_norm, (size_t)t * K * 4, (size_t)K * 4);
            ds3_metal_buffer_t *lv = ds3_metal_buffer_view(b_logits, (size_t)t * E * 4, (size_t)E * 4);
            CHECK(nv && lv);
            CHECK(ds3_metal_moe_ffn_router(nv, router, lv, K, E, rs, DS3_HIP_TYPE_F32) == 0);
            ds3_metal_buffer_free(nv);
            ds3_metal_buffer_free(lv);
        }
        CHECK(ds3_metal_begin_batch() == 0);
        CHECK(ds3_metal_moe_router_topk_batch_tokens(b_logits, b_idx, b_sc, 1, M, E, k, true) == 0);
        ds3_metal_end_batch();
        CHECK(ds3_metal_buffer_read(b_idx, 0, idx_all, (size_t)M * k * 4) == 0);
        CHECK(ds3_metal_buffer_read(b_sc, 0, sc_all, (size_t)M * k * 4) == 0);
        CHECK(ds3_metal_buffer_zero_f32(b_ffn, (size_t)M * K * 4) == 0);

        /* host bucketing in token order, expert-major with stride M */
        unsigned *counts = calloc(E, sizeof(unsigned));
        int32_t *ids_h = malloc((size_t)E * M * 4);
        float *gsc_h = malloc((size_t)E * M * 4);
        CHECK(counts && ids_h && gsc_h);
        for (unsigned t = 0; t < M; t++)
            for (unsigned j = 0; j < k; j++) {
                const int ex = idx_all[(size_t)t * k + j];
                CHECK(ex >= 0 && (unsigned)ex < E);
                const size_t at = (size_t)ex * M + counts[ex]++;
                ids_h[at] = (int32_t)t;
                gsc_h[at] = sc_all[(size_t)t * k + j];
            }
        CHECK(ds3_metal_buffer_write(b_gids, 0, ids_h, (size_t)E * M * 4) == 0);
        CHECK(ds3_metal_buffer_write(b_gsc, 0, gsc_h, (size_t)E * M * 4) == 0);
        for (unsigned ex = 0; ex < E; ex++) {
            const unsigned c = counts[ex];
            if (c == 0) continue;
            CHECK(ds3_metal_gather_rows_f32(b_norm, b_gids, b_md, K, c, ex * M) == 0);
            CHECK(ds3_metal_matmul_quantized_batch(b_md, gate, b_mh, c, F, K, gs, (uint64_t)ex * F * gs, gt) == 0);
            CHECK(ds3_metal_matmul_quantized_batch(b_md, up, b_mu, c, F, K, us, (uint64_t)ex * F * us, ut) == 0);
            CHECK(ds3_metal_silu_mul_f32(b_mh, b_mu, b_mu, c * F) == 0);
            CHECK(ds3_metal_matmul_quantized_batch(b_mu, down, b_md, c, K, F, ds, (uint64_t)ex * K * ds, dt) == 0);
            CHECK(ds3_metal_scatter_add_weighted_f32(b_md, b_gsc, b_gids, b_ffn, K, c, ex * M) == 0);
        }
        CHECK(ds3_metal_vec_add(b_ffn, b_res, b_hidden, M * K) == 0);
        CHECK(ds3_metal_buffer_read(b_hidden, 0, out, (size_t)M * K * 4) == 0);
        CHECK(write_file(dir, "prefill_out.f32", out, (size_t)M * K * 4) == 0);
        CHECK(write_file(dir, "prefill_idx.i32", idx_all, (size_t)M * k * 4) == 0);
        free(counts);
        free(ids_h);
        free(gsc_h);
        ds3_metal_buffer_t *bs[] = { b_hidden, b_norm, b_res, b_ffn, b_logits, b_idx, b_sc, b_gids, b_gsc, b_mh, b_mu, b_md };
        for (size_t i = 0; i < sizeof bs / sizeof bs[0]; i++) ds3_metal_buffer_free(bs[i]);
    }

    /* ------------------------------------------------ gpu-only decode (moe_ffn) */
    {
        /* the engine's [E][3] expert offset table (src/ds3_engine.c:1747-1773) */
        uint64_t *tbl = malloc((size_t)E * 3 * sizeof(uint64_t));
        CHECK(tbl != NULL);
        for (unsigned e = 0; e < E; e++) {
            tbl[3 * e + 0] = (uint64_t)e * F * gs;
            tbl[3 * e + 1] = (uint64_t)e * F * us;
            tbl[3 * e + 2] = (uint64_t)e * K * ds;
        }
        ds3_metal_buffer_t *b_tbl = ds3_metal_buffer_alloc((size_t)E * 3 * sizeof(uint64_t));
        ds3_metal_buffer_t *b_hidden = ds3_metal_buffer_alloc((size_t)K * 4);
        ds3_metal_buffer_t *b_norm = ds3_metal_buffer_alloc((size_t)K * 4);
        ds3_metal_buffer_t *b_res = ds3_metal_buffer_alloc((size_t)K * 4);
        ds3_metal_buffer_t *b_ffn = ds3_metal_buffer_alloc((size_t)K * 4);
        ds3_metal_buffer_t *b_logits = ds3_metal_buffer_alloc((size_t)E * 4);
        ds3_metal_buffer_t *b_mh = ds3_metal_buffer_alloc((size_t)k * F * 4);
        ds3_metal_buffer_t *b_mu = ds3_metal_buffer_alloc((size_t)k * F * 4);
        ds3_metal_buffer_t *b_md = ds3_metal_buffer_alloc((size_t)k * K * 4);
        CHECK(b_tbl && b_hidden && b_norm && b_res && b_ffn && b_logits && b_mh && b_mu && b_md);
        CHECK(ds3_metal_buffer_write(b_tbl, 0, tbl, (size_t)E * 3 * sizeof(uint64_t)) == 0);
        for (unsigned t = 0; t < T; t++) {
            CHECK(ds3_metal_buffer_write(b_hidden, 0, hidden + (size_t)t * K, (size_t)K * 4) == 0);
            CHECK(ds3_metal_buffer_write(b_res, 0, residual + (size_t)t * K, (size_t)K * 4) == 0);
            CHECK(ds3_metal_rms_norm(b_hidden, b_ffn_norm, b_norm, K, 1, NORM_EPS) == 0);
            CHECK(ds3_metal_buffer_zero_f32(b_ffn, (size_t)K * 4) == 0);
            CHECK(ds3_metal_moe_ffn(b_norm, router, gate, up, down, gt, ut, dt, gs, us, ds, NULL, NULL, NULL,
                                    DS3_HIP_TYPE_F32, DS3_HIP_TYPE_F32, DS3_HIP_TYPE_F32, 0, 0, 0, b_ffn, b_logits,
                                    b_tbl, b_mh, b_mu, b_md, K, E, k, F, 0, rs, DS3_HIP_TYPE_F32, true) == 0);
            CHECK(ds3_metal_vec_add(b_ffn, b_res, b_hidden, K) == 0);
            CHECK(ds3_metal_buffer_read(b_hidden, 0, out + (size_t)t * K, (size_t)K * 4) == 0);
        }
        CHECK(write_file(dir, "gpuonly_out.f32", out, (size_t)T * K * 4) == 0);
        ds3_metal_buffer_t *bs[] = { b_tbl, b_hidden, b_norm, b_res, b_ffn, b_logits, b_mh, b_mu, b_md };
        for (size_t i = 0; i < sizeof bs / sizeof bs[0]; i++) ds3_metal_buffer_free(bs[i]);
        free(tbl);
    }

    /* --------------------------------------- block per token, then as one graph */
    {
        ds3_metal_buffer_t *b_hid = ds3_metal_buffer_alloc((size_t)T * K * 4);
        ds3_metal_buffer_t *b_idx = ds3_metal_buffer_alloc((size_t)T * k * 4);
        CHECK(b_hid && b_idx);
        ds3_metal_buffer_t *hv[256], *iv[256];
        CHECK(T <= 256);
        for (unsigned t = 0; t < T; t++) {
            hv[t] = ds3_metal_buffer_view(b_hid, (size_t)t * K * 4, (size_t)K * 4);
            iv[t] = ds3_metal_buffer_view(b_idx, (size_t)t * k * 4, (size_t)k * 4);
            CHECK(hv[t] && iv[t]);
        }
        CHECK(ds3_metal_buffer_write(b_hid, 0, hidden, (size_t)T * K * 4) == 0);
        for (unsigned t = 0; t < T; t++)
            CHECK(ds3_hip_moe_block(hv[t], b_ffn_norm, NORM_EPS, router, gate, up, down, gt, ut, dt, gs, us, ds, NULL,
                                    NULL, NULL, iv[t], NULL, 1, K, E, k, F, rs, DS3_HIP_TYPE_F32, true) == 0);
        CHECK(ds3_metal_buffer_read(b_hid, 0, out, (size_t)T * K * 4) == 0);
        CHECK(ds3_metal_buffer_read(b_idx, 0, idx_all, (size_t)T * k * 4) == 0);
        CHECK(write_file(dir, "block_out.f32", out, (size_t)T * K * 4) == 0);
        CHECK(write_file(dir, "block_idx.i32", idx_all, (size_t)T * k * 4) == 0);
        /* the same calls captured once and replayed on the same input */
        void *graph = NULL;
        CHECK(ds3_hip_graph_begin() == 0);
        for (unsigned t = 0; t < T; t++)
            CHECK(ds3_hip_moe_block(hv[t], b_ffn_norm, NORM_EPS, router, gate, up, down, gt, ut, dt, gs, us, ds, NULL,
                                    NULL, NULL, iv[t], NULL, 1, K, E, k, F, rs, DS3_HIP_TYPE_F32, true) == 0);
        CHECK(ds3_hip_graph_end(&graph) == 0 && graph != NULL);
        CHECK(ds3_metal_buffer_write(b_hid, 0, hidden, (size_t)T * K * 4) == 0);
        CHECK(ds3_hip_graph_launch(graph) == 0);
        CHECK(ds3_metal_buffer_read(b_hid, 0, out, (size_t)T * K * 4) == 0);
        CHECK(write_file(dir, "graph_out.f32", out, (size_t)T * K * 4) == 0);
        ds3_hip_graph_destroy(graph);
        for (unsigned t = 0; t < T; t++) {
            ds3_metal_buffer_free(hv[t]);
            ds3_metal_buffer_free(iv[t]);
        }
        ds3_metal_buffer_free(b_hid);
        ds3_metal_buffer_free(b_idx);
    }

    /* ------------------------------------------- prefill chunk in one batch call */
    {
        const unsigned M = T;
        ds3_metal_buffer_t *b_hidden = ds3_metal_buffer_alloc((size_t)M * K * 4);
        ds3_metal_buffer_t *b_norm = ds3_metal_buffer_alloc((size_t)M * K * 4);
        ds3_metal_buffer_t *b_res = ds3_metal_buffer_alloc((size_t)M * K * 4);
        ds3_metal_buffer_t *b_ffn = ds3_metal_buffer_alloc((size_t)M * K * 4);
        ds3_metal_buffer_t *b_idx = ds3_metal_buffer_alloc((size_t)M * k * 4);
        CHECK(b_hidden && b_norm && b_res && b_ffn && b_idx);
        CHECK(ds3_metal_buffer_write(b_hidden, 0, hidden, (size_t)M * K * 4) == 0);
        CHECK(ds3_metal_buffer_write(b_res, 0, residual, (size_t)M * K * 4) == 0);
        CHECK(ds3_metal_rms_norm(b_hidden, b_ffn_norm, b_norm, K, M, NORM_EPS) == 0);
        CHECK(ds3_metal_buffer_zero_f32(b_ffn, (size_t)M * K * 4) == 0);
        CHECK(ds3_hip_moe_ffn_batch(b_norm, router, gate, up, down, gt, ut, dt, gs, us, ds, NULL, b_ffn, b_res, NULL,
                                    b_idx, NULL, M, K, E, k, F, rs, DS3_HIP_TYPE_F32, true) == 0);
        CHECK(ds3_metal_buffer_read(b_ffn, 0, out, (size_t)M * K * 4) == 0);
        CHECK(ds3_metal_buffer_read(b_idx, 0, idx_all, (size_t)M * k * 4) == 0);
        CHECK(write_file(dir, "batch_out.f32", out, (size_t)M * K * 4) == 0);
        CHECK(write_file(dir, "batch_idx.i32", idx_all, (size_t)M * k * 4) == 0);
        ds3_metal_buffer_t *bs[] = { b_hidden, b_norm, b_res, b_ffn, b_idx };
        for (size_t i = 0; i < sizeof bs / sizeof bs[0]; i++) ds3_metal_buffer_free(bs[i]);
    }

    ds3_metal_buffer_free(router);
    ds3_metal_buffer_free(gate);
    ds3_metal_buffer_free(up);
    ds3_metal_buffer_free(down);
    ds3_metal_buffer_free(wbuf);
    ds3_metal_buffer_free(b_ffn_norm);
    munmap(map, blob);
    ds3_metal_shutdown();
    free(hidden);
    free(gain);
    free(residual);
    free(out);
    free(norm_rows);
    free(idx_all);
    free(sc_all);
    fprintf(stderr, "engine_sequences: decode, prefill, gpu-only, block, graph and batch done, T=%u E=%u\n", T, E);
    return 0;
}
