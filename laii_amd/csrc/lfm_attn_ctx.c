/*
 * lfm_attn_ctx.c -- C11 engine context: device-resident KV caches, RoPE
 * tables and QK-norm weights per attention layer, and the host-pointer
 * attention step the forward stacks call (include/lfm_attn.h).
 *
 * Each step stages q | k | v | gate | position in one pinned host buffer,
 * moves it with a single host-to-device copy, runs the attention kernel with
 * the prologue fused (QK-RMSNorm + RoPE, RNE fp16 K/V store at the
 * position's slot, lfm_hip_gqa_f16_step), and returns the output with a
 * single device-to-host copy, all on the context's stream.
 */
#define _POSIX_C_SOURCE 200809L /* getpid, fsync, fileno */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "lfm_attn.h"

#define LFM_CTX_MAX_ROWS 8u /* LFM2_MAX_BATCH, tools/lfm2_prefill_batch.c:88 */

struct lfm_attn_ctx {
    lfm_attn_geom g;
    uint8_t *is_swa;      /* [n_layers] */
    uint32_t *slots;      /* [n_layers] cache rows */
    uint16_t **k_cache;   /* [n_layers] device */
    uint16_t **v_cache;
    float **q_norm;       /* [n_layers] device or NULL */
    float **k_norm;
    uint16_t **tables;    /* device: [n_layers][2] {k_cache, v_cache} pointer pairs */
    float *cos_full, *sin_full, *cos_swa, *sin_swa; /* device LUTs [max_seq][hd/2] */
    float *cos_shift, *sin_shift; /* LFM_PROLOGUE_TABLE: the lfm2_rope_lut_init table
                                     for sink eviction (else the full-layer table) */
    unsigned char *stage_host;  /* pinned: q | k | v | gate | pos | out */
    unsigned char *stage_dev;
    size_t off_k, off_v, off_g, off_pos, off_out, stage_in_bytes, out_bytes;
    unsigned char *pf_host;     /* pinned: prefill q | k | v | pos in, out (grown on demand) */
    unsigned char *pf_dev;      /* device: the same plus fp16 q */
    size_t pf_host_bytes, pf_dev_bytes;
    unsigned char *file_host;   /* pinned: a whole .lfmcache file (grown on demand) */
    unsigned char *file_dev;    /* its payload in device memory */
    size_t file_host_bytes, file_dev_bytes;
    hipStream_t stream;
};

static int st_of(hipError_t e) {
    if (e == hipSuccess) return LFM_ATTN_OK;
    return e == hipErrorOutOfMemory ? LFM_ATTN_E_NOMEM : LFM_ATTN_E_DEVICE;
}

static size_t align256(size_t x) { return (x + 255u) & ~(size_t)255u; }

void lfm_attn_ctx_destroy(lfm_attn_ctx *c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (uint32_t l = 0; c->k_cache && l < c->g.n_layers; ++l) {
        (void)hipFree(c->k_cache[l]);
        (void)hipFree(c->v_cache[l]);
        if (c->q_norm) (void)hipFree(c->q_norm[l]);
        if (c->k_norm) (void)hipFree(c->k_norm[l]);
    }
    (void)hipFree(c->tables);
    (void)hipFree(c->cos_full);
    (void)hipFree(c->sin_full);
    (void)hipFree(c->cos_swa);
    (void)hipFree(c->sin_swa);
    if (c->cos_shift != c->cos_full) (void)hipFree(c->cos_shift);
    if (c->sin_shift != c->sin_full) (void)hipFree(c->sin_shift);
    (void)hipFree(c->stage_dev);
    if (c->stage_host) (void)hipHostFree(c->stage_host);
    (void)hipFree(c->file_dev);
    if (c->file_host) (void)hipHostFree(c->file_host);
    (void)hipFree(c->pf_dev);
    if (c->pf_host) (void)hipHostFree(c->pf_host);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    free(c->is_swa);
    free(c->slots);
    free(c->k_cache);
    free(c->v_cache);
    free(c->q_norm);
    free(c->k_norm);
    free(c);
}

/* Build a RoPE table on the host (bit-identical to the reference builders)
 * and upload it.  which: 0 the full-layer table of the geometry's prologue,
 * 1 the SWA table, 2 the lfm2_rope_lut_init table (LFM2 sink eviction). */
static int upload_lut(lfm_attn_ctx *c, int which, float **cos_d, float **sin_d) {
    const lfm_attn_geom *g = &c->g;
    const size_t n = (size_t)g->max_seq * (g->head_dim / 2u);
    float *hc = (float *)malloc(n * sizeof(float));
    float *hs = (float *)malloc(n * sizeof(float));
    int st = (hc && hs) ? LFM_ATTN_OK : LFM_ATTN_E_NOMEM;
    const int swa = which == 1;
    if (st == LFM_ATTN_OK) {
        if (!g->lfm3 && which == 0 && g->prologue == LFM_PROLOGUE_TABLE)
            st = lfm_attn_rope_table_lfm2(hc, hs, g->max_seq, g->head_dim, g->rope_base);
        else if (!g->lfm3)
            st = lfm_attn_rope_lut_lfm2(hc, hs, g->max_seq, g->head_dim, g->rope_base);
        else if (swa) /* tools/lfm3_engine.c:1720-1723: full rotation, no rope_freqs */
            st = lfm_attn_rope_lut_lfm3(hc, hs, g->max_seq, g->head_dim, g->head_dim,
                                        g->rope_base_swa, NULL, 0);
        else
            st = lfm_attn_rope_lut_lfm3(hc, hs, g->max_seq, g->head_dim, g->rope_dim,
                                        g->rope_base, g->rope_freqs, g->n_rope_freqs);
    }
    if (st == LFM_ATTN_OK) st = st_of(hipMalloc((void **)cos_d, n * sizeof(float)));
    if (st == LFM_ATTN_OK) st = st_of(hipMalloc((void **)sin_d, n * sizeof(float)));
    if (st == LFM_ATTN_OK) st = st_of(hipMemcpy(*cos_d, hc, n * sizeof(float), hipMemcpyHostToDevice));
    if (st == LFM_ATTN_OK) st = st_of(hipMemcpy(*sin_d, hs, n * sizeof(float), hipMemcpyHostToDevice));
    free(hc);
    free(hs);
    return st;
}

int lfm_attn_ctx_create(lfm_attn_ctx **out, const lfm_attn_geom *geom) {
    if (!out || !geom) return LFM_ATTN_E_INVALID;
    *out = NULL;
    const lfm_attn_geom *g = geom;
    if (g->n_layers == 0u || g->n_head_q == 0u || g->n_head_kv == 0u ||
        g->n_head_q % g->n_head_kv != 0u || g->head_dim == 0u || g->head_dim % 8u != 0u ||
        g->head_dim > 256u || g->max_seq == 0u || g->max_seq >= 0x7FFFFFFFu)
        return LFM_ATTN_E_INVALID;
    if (g->prologue != LFM_PROLOGUE_FAST && (g->prologue != LFM_PROLOGUE_TABLE || g->lfm3)) return LFM_ATTN_E_INVALID;
    int any_swa = 0;
    for (uint32_t l = 0; g->layer_is_swa && l < g->n_layers; ++l) any_swa |= g->layer_is_swa[l] != 0;
    /* a step of LFM_CTX_MAX_ROWS rows writes that many ring slots while its
     * first row's window is still read: the ring holds window + 7 slots or
     * more (the engines use window + 8, tools/lfm3_engine.c:1673) */
    if (any_swa && (g->sliding_window == 0u || (uint64_t)g->swa_cap < (uint64_t)g->sliding_window + LFM_CTX_MAX_ROWS - 1u))
        return LFM_ATTN_E_INVALID;

    lfm_attn_ctx *c = (lfm_attn_ctx *)calloc(1, sizeof *c);
    if (!c) return LFM_ATTN_E_NOMEM;
    c->g = *g;
    c->g.layer_is_swa = NULL;
    c->g.rope_freqs = NULL; /* only used while building the table below */
    const uint32_t L = g->n_layers;
    c->is_swa  = (uint8_t *)calloc(L, 1);
    c->slots   = (uint32_t *)calloc(L, sizeof(uint32_t));
    c->k_cache = (uint16_t **)calloc(L, sizeof(uint16_t *));
    c->v_cache = (uint16_t **)calloc(L, sizeof(uint16_t *));
    c->q_norm  = (float **)calloc(L, sizeof(float *));
    c->k_norm  = (float **)calloc(L, sizeof(float *));
    int st = (c->is_swa && c->slots && c->k_cache && c->v_cache && c->q_norm && c->k_norm)
                 ? LFM_ATTN_OK : LFM_ATTN_E_NOMEM;
    if (st == LFM_ATTN_OK) st = st_of(hipStreamCreate(&c->stream));
    const size_t kv_dim = (size_t)g->n_head_kv * g->head_dim;
    uint16_t **host_tables = (uint16_t **)calloc(2u * L, sizeof(uint16_t *));
    if (!host_tables && st == LFM_ATTN_OK) st = LFM_ATTN_E_NOMEM;
    for (uint32_t l = 0; st == LFM_ATTN_OK && l < L; ++l) {
        c->is_swa[l] = (g->layer_is_swa && g->layer_is_swa[l]) ? 1u : 0u;
        c->slots[l]  = c->is_swa[l] ? g->swa_cap : g->max_seq;
        const size_t bytes = (size_t)c->slots[l] * kv_dim * sizeof(uint16_t);
        st = st_of(hipMalloc((void **)&c->k_cache[l], bytes));
        if (st == LFM_ATTN_OK) st = st_of(hipMalloc((void **)&c->v_cache[l], bytes));
        if (st == LFM_ATTN_OK) st = st_of(hipMemset(c->k_cache[l], 0, bytes));
        if (st == LFM_ATTN_OK) st = st_of(hipMemset(c->v_cache[l], 0, bytes));
        host_tables[2u * l]      = c->k_cache[l];
        host_tables[2u * l + 1u] = c->v_cache[l];
    }
    if (st == LFM_ATTN_OK) st = st_of(hipMalloc((void **)&c->tables, 2u * L * sizeof(uint16_t *)));
    if (st == LFM_ATTN_OK)
        st = st_of(hipMemcpy(c->tables, host_tables, 2u * L * sizeof(uint16_t *), hipMemcpyHostToDevice));
    free(host_tables);
    if (st == LFM_ATTN_OK) {
        lfm_attn_geom full = *g; /* rope_freqs still points at the caller's factors here */
        lfm_attn_geom saved = c->g;
        c->g = full;
        st = upload_lut(c, 0, &c->cos_full, &c->sin_full);
        if (st == LFM_ATTN_OK && any_swa) st = upload_lut(c, 1, &c->cos_swa, &c->sin_swa);
        if (st == LFM_ATTN_OK && g->prologue == LFM_PROLOGUE_TABLE) {
            st = upload_lut(c, 2, &c->cos_shift, &c->sin_shift);
        } else {
            c->cos_shift = c->cos_full;
            c->sin_shift = c->sin_full;
        }
        c->g = saved;
    }
    /* staging: q | k | v | gate | pos, then out */
    const size_t R = LFM_CTX_MAX_ROWS;
    c->off_k          = align256(R * g->n_head_q * g->head_dim * sizeof(float));
    c->off_v          = c->off_k + align256(R * kv_dim * sizeof(float));
    c->off_g          = c->off_v + align256(R * kv_dim * sizeof(float));
    c->off_pos        = c->off_g + align256(R * g->n_head_q * sizeof(float));
    c->stage_in_bytes = c->off_pos + align256(sizeof(uint32_t));
    c->off_out        = c->stage_in_bytes;
    c->out_bytes      = R * g->n_head_q * g->head_dim * sizeof(float);
    if (st == LFM_ATTN_OK)
        st = st_of(hipHostMalloc((void **)&c->stage_host, c->off_out + c->out_bytes, hipHostMallocDefault));
    if (st == LFM_ATTN_OK) st = st_of(hipMalloc((void **)&c->stage_dev, c->off_out + c->out_bytes));
    if (st != LFM_ATTN_OK) {
        lfm_attn_ctx_destroy(c);
        return st;
    }
    *out = c;
    return LFM_ATTN_OK;
}

int lfm_attn_ctx_set_norms(lfm_attn_ctx *c, uint32_t layer, const float *q_norm_w,
                           const float *k_norm_w) {
    if (!c || layer >= c->g.n_layers) return LFM_ATTN_E_INVALID;
    const size_t bytes = (size_t)c->g.head_dim * sizeof(float);
    const float *src[2] = {q_norm_w, k_norm_w};
    float **dst[2]      = {&c->q_norm[layer], &c->k_norm[layer]};
    for (int i = 0; i < 2; ++i) {
        if (!src[i]) {
            (void)hipFree(*dst[i]);
            *dst[i] = NULL;
            continue;
        }
        if (!*dst[i]) {
            int st = st_of(hipMalloc((void **)dst[i], bytes));
            if (st != LFM_ATTN_OK) return st;
        }
        int st = st_of(hipMemcpy(*dst[i], src[i], bytes, hipMemcpyHostToDevice));
        if (st != LFM_ATTN_OK) return st;
    }
    return LFM_ATTN_OK;
}

int lfm_attn_ctx_forward(lfm_attn_ctx *c, uint32_t layer, uint32_t pos_0, uint32_t B,
                         const float *q, const float *k, const float *v,
                         const float *gate_logits, float *out) {
    if (!c || !q || !k || !v || !out || layer >= c->g.n_layers) return LFM_ATTN_E_INVALID;
    if (B == 0u || B > LFM_CTX_MAX_ROWS) return LFM_ATTN_E_INVALID;
    const lfm_attn_geom *g = &c->g;
    if ((uint64_t)pos_0 + B > g->max_seq) return LFM_ATTN_E_RANGE;
    const int swa = c->is_swa[layer];
    const uint32_t window = swa ? g->sliding_window : 0u;
    const uint32_t cap    = c->slots[layer];
    /* every row's window must survive the later rows' ring writes */
    if (swa && (uint64_t)window + B - 1u > cap) return LFM_ATTN_E_INVALID;

    const size_t qn = (size_t)B * g->n_head_q * g->head_dim;
    const size_t kn = (size_t)B * g->n_head_kv * g->head_dim;
    unsigned char *h = c->stage_host;
    memcpy(h, q, qn * sizeof(float));
    memcpy(h + c->off_k, k, kn * sizeof(float));
    memcpy(h + c->off_v, v, kn * sizeof(float));
    if (gate_logits) memcpy(h + c->off_g, gate_logits, (size_t)B * g->n_head_q * sizeof(float));
    memcpy(h + c->off_pos, &pos_0, sizeof pos_0);
    int st = st_of(hipMemcpyAsync(c->stage_dev, h, c->stage_in_bytes, hipMemcpyHostToDevice, c->stream));
    if (st != LFM_ATTN_OK) return st;

    unsigned char *d     = c->stage_dev;
    const float *qd      = (const float *)d;
    const uint32_t *posd = (const uint32_t *)(d + c->off_pos);
    uint16_t *const *kt  = c->tables + 2u * layer;
    uint16_t *const *vt  = c->tables + 2u * layer + 1u;
    const float *cosd    = swa ? c->cos_swa : c->cos_full;
    const float *sind    = swa ? c->sin_swa : c->sin_full;
    /* one launch: QK-norm + RoPE, the fp16 K/V store and the attention
     * (plus the split merge when the keys are split) */
    const uint32_t keys = window ? window + B - 1u : pos_0 + B;
    st = lfm_hip_gqa_f16_step(qd, (const float *)(d + c->off_k), (const float *)(d + c->off_v),
                              gate_logits ? (const float *)(d + c->off_g) : NULL, 1, kt, vt, posd,
                              (float *)(d + c->off_out), 1u, B, keys, g->n_head_q, g->n_head_kv, g->head_dim,
                              window, cap, 1.0f / sqrtf((float)g->head_dim), c->q_norm[layer], c->k_norm[layer],
                              g->eps, cosd, sind, g->prologue, c->stream);
    if (st != LFM_ATTN_OK) return st;
    st = st_of(hipMemcpyAsync(h + c->off_out, d + c->off_out, qn * sizeof(float),
                              hipMemcpyDeviceToHost, c->stream));
    if (st == LFM_ATTN_OK) st = st_of(hipStreamSynchronize(c->stream));
    if (st == LFM_ATTN_OK) memcpy(out, h + c->off_out, qn * sizeof(float));
    return st;
}

/* Prompt prefill of one layer in one attention launch (after one prologue
 * launch), where lfm2_forward_batch / lfm3_forward_batch_core run the layer
 * LFM2_MAX_BATCH rows at a time (tools/lfm2_prefill_batch.c:1129-1199,
 * tools/lfm3_engine.c:1918-2055):
 *  - full-attention layers: the prologue writes every row's K/V into the
 *    cache, then every row attends keys 0 .. its position (head_dim 64
 *    without a gate: lfm_hip_prefill_f16; head_dim 128, gated or not:
 *    lfm_hip_lfm3_prefill_f16);
 *  - sliding-window layers (head_dim 128): the ring of window + 8 slots
 *    cannot hold a whole prompt, so the window before the prompt (positions
 *    kv_pos0 .. pos_0 - 1, at most window - 1 of them) is copied from the
 *    ring into a linear buffer, the prologue appends the prompt's rows, the
 *    prefill reads the buffer (row r = position kv_pos0 + r), and the last
 *    min(n_rows, cap) rows are copied back to their ring slots -- the ring
 *    then holds what the chunked steps leave in it.
 * The prologue addresses the buffer with positions relative to kv_pos0 and
 * RoPE tables offset by kv_pos0 rows, so every row is rotated with its
 * absolute position.  Other shapes, and prompts of at most 8 rows, run the
 * step over chunks of LFM_CTX_MAX_ROWS rows. */
static int ring_copy(uint16_t *dst, size_t dst_row, const uint16_t *src, size_t src_row, uint32_t n, size_t row_elems,
                     hipStream_t stream) {
    return st_of(hipMemcpyAsync(dst + dst_row * row_elems, src + src_row * row_elems,
                                (size_t)n * row_elems * sizeof(uint16_t), hipMemcpyDeviceToDevice, stream));
}

/* positions p0 .. p0 + n - 1: ring slots p % cap <-> linear rows p - base */
static int ring_move(lfm_attn_ctx *c, uint32_t layer, uint16_t *lin_k, uint16_t *lin_v, uint32_t base, uint32_t p0,
                     uint32_t n, int to_ring) {
    const uint32_t cap = c->slots[layer];
    const size_t row   = (size_t)c->g.n_head_kv * c->g.head_dim;
    uint32_t done = 0;
    int st = LFM_ATTN_OK;
    while (st == LFM_ATTN_OK && done < n) {
        const uint32_t slot = (p0 + done) % cap;
        const uint32_t run  = (n - done < cap - slot) ? n - done : cap - slot;
        const uint32_t lrow = p0 + done - base;
        if (to_ring) {
            st = ring_copy(c->k_cache[layer], slot, lin_k, lrow, run, row, c->stream);
            if (st == LFM_ATTN_OK) st = ring_copy(c->v_cache[layer], slot, lin_v, lrow, run, row, c->stream);
        } else {
            st = ring_copy(lin_k, lrow, c->k_cache[layer], slot, run, row, c->stream);
            if (st == LFM_ATTN_OK) st = ring_copy(lin_v, lrow, c->v_cache[layer], slot, run, row, c->stream);
        }
        done += run;
    }
    return st;
}

int lfm_attn_ctx_prefill(lfm_attn_ctx *c, uint32_t layer, uint32_t pos_0, uint32_t n_rows, const float *q,
                         const float *k, const float *v, const float *gate_logits, float *out) {
    if (!c || !q || !k || !v || !out || layer >= c->g.n_layers || n_rows == 0u) return LFM_ATTN_E_INVALID;
    const lfm_attn_geom *g = &c->g;
    if ((uint64_t)pos_0 + n_rows > g->max_seq) return LFM_ATTN_E_RANGE;
    const uint32_t kv_mul = g->n_head_q / g->n_head_kv;
    const size_t qrow = (size_t)g->n_head_q * g->head_dim, krow = (size_t)g->n_head_kv * g->head_dim;
    const int swa = c->is_swa[layer];
    const int mfma64 = !swa && !gate_logits && g->head_dim == 64u && kv_mul <= 16u && (256u % kv_mul) == 0u;
    const int mfma128 = g->head_dim == 128u && kv_mul <= 32u && (128u % kv_mul) == 0u;
    if (n_rows <= LFM_CTX_MAX_ROWS || !(mfma64 || mfma128)) {
        for (uint32_t r = 0; r < n_rows; r += LFM_CTX_MAX_ROWS) {
            const uint32_t b = n_rows - r < LFM_CTX_MAX_ROWS ? n_rows - r : LFM_CTX_MAX_ROWS;
            const int st = lfm_attn_ctx_forward(c, layer, pos_0 + r, b, q + r * qrow, k + r * krow, v + r * krow,
                                                gate_logits ? gate_logits + (size_t)r * g->n_head_q : NULL,
                                                out + r * qrow);
            if (st != LFM_ATTN_OK) return st;
        }
        return LFM_ATTN_OK;
    }
    const uint32_t window = swa ? g->sliding_window : 0u;
    const uint32_t n_old  = swa ? (pos_0 < window - 1u ? pos_0 : window - 1u) : 0u;
    const uint32_t kv_pos0 = pos_0 - n_old; /* position of linear row 0 (sliding window) */
    const uint32_t rel_pos = swa ? n_old : pos_0;
    /* device layout: q f32 | k f32 | v f32 | gate f32 | pos + pointer pair,
     * out f32, then (sliding window) the linear K and V buffers */
    const size_t qb = align256((size_t)n_rows * qrow * sizeof(float));
    const size_t kb = align256((size_t)n_rows * krow * sizeof(float));
    const size_t gb = gate_logits ? align256((size_t)n_rows * g->n_head_q * sizeof(float)) : 0u;
    const size_t pb = 256u;
    const size_t in_bytes = qb + 2u * kb + gb + pb;
    const size_t lin_bytes = swa ? align256((size_t)(n_old + n_rows) * krow * sizeof(uint16_t)) : 0u;
    const size_t dev_bytes = in_bytes + qb + 2u * lin_bytes;
    int st = LFM_ATTN_OK;
    if (c->pf_host_bytes < in_bytes + qb) {
        if (c->pf_host) (void)hipHostFree(c->pf_host);
        c->pf_host = NULL;
        c->pf_host_bytes = 0;
        st = st_of(hipHostMalloc((void **)&c->pf_host, in_bytes + qb, hipHostMallocDefault));
        if (st != LFM_ATTN_OK) return st;
        c->pf_host_bytes = in_bytes + qb;
    }
    if (c->pf_dev_bytes < dev_bytes) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(c->pf_dev);
        c->pf_dev = NULL;
        c->pf_dev_bytes = 0;
        st = st_of(hipMalloc((void **)&c->pf_dev, dev_bytes));
        if (st != LFM_ATTN_OK) return st;
        c->pf_dev_bytes = dev_bytes;
    }
    unsigned char *h = c->pf_host, *d = c->pf_dev;
    const size_t off_k = qb, off_v = qb + kb, off_g = qb + 2u * kb, off_p = off_g + gb;
    uint16_t *lin_k = swa ? (uint16_t *)(d + in_bytes + qb) : NULL;
    uint16_t *lin_v = swa ? (uint16_t *)(d + in_bytes + qb + lin_bytes) : NULL;
    memcpy(h, q, (size_t)n_rows * qrow * sizeof(float));
    memcpy(h + off_k, k, (size_t)n_rows * krow * sizeof(float));
    memcpy(h + off_v, v, (size_t)n_rows * krow * sizeof(float));
    if (gate_logits) memcpy(h + off_g, gate_logits, (size_t)n_rows * g->n_head_q * sizeof(float));
    memcpy(h + off_p, &rel_pos, sizeof rel_pos);
    uint16_t *pair[2] = {lin_k, lin_v};
    memcpy(h + off_p + 16u, pair, sizeof pair);
    st = st_of(hipMemcpyAsync(d, h, in_bytes, hipMemcpyHostToDevice, c->stream));
    if (st != LFM_ATTN_OK) return st;
    float *qd = (float *)d;
    float *od = (float *)(d + in_bytes);
    const float *gd = gate_logits ? (const float *)(d + off_g) : NULL;
    const float scale = 1.0f / sqrtf((float)g->head_dim);
    const size_t half = g->head_dim / 2u;
    if (swa) {
        uint16_t *const *lin_t = (uint16_t *const *)(d + off_p + 16u);
        st = ring_move(c, layer, lin_k, lin_v, kv_pos0, kv_pos0, n_old, 0);
        if (st == LFM_ATTN_OK)
            st = lfm_hip_qkv_prologue(qd, (const float *)(d + off_k), (const float *)(d + off_v), lin_t, lin_t + 1,
                                      (const uint32_t *)(d + off_p), 1u, n_rows, g->n_head_q, g->n_head_kv,
                                      g->head_dim, c->q_norm[layer], c->k_norm[layer], g->eps,
                                      c->cos_swa + (size_t)kv_pos0 * half, c->sin_swa + (size_t)kv_pos0 * half, 0u,
                                      0u, g->prologue, c->stream);
        if (st == LFM_ATTN_OK)
            st = lfm_hip_lfm3_prefill_f16(qd, lin_k, lin_v, gd, 1, od, 1u, n_rows, pos_0, kv_pos0, 0u, window,
                                          g->n_head_q, g->n_head_kv, g->head_dim, scale, c->stream);
        const uint32_t cap = c->slots[layer];
        const uint32_t n_back = n_rows < cap ? n_rows : cap;
        if (st == LFM_ATTN_OK) st = ring_move(c, layer, lin_k, lin_v, kv_pos0, pos_0 + n_rows - n_back, n_back, 1);
    } else {
        st = lfm_hip_qkv_prologue(qd, (const float *)(d + off_k), (const float *)(d + off_v), c->tables + 2u * layer,
                                  c->tables + 2u * layer + 1u, (const uint32_t *)(d + off_p), 1u, n_rows,
                                  g->n_head_q, g->n_head_kv, g->head_dim, c->q_norm[layer], c->k_norm[layer], g->eps,
                                  c->cos_full, c->sin_full, 0u, 0u, g->prologue, c->stream);
        if (st == LFM_ATTN_OK && mfma128)
            st = lfm_hip_lfm3_prefill_f16(qd, c->k_cache[layer], c->v_cache[layer], gd, 1, od, 1u, n_rows, pos_0, 0u,
                                          0u, 0u, g->n_head_q, g->n_head_kv, g->head_dim, scale, c->stream);
        else if (st == LFM_ATTN_OK)
            st = lfm_hip_prefill_f16(qd, c->k_cache[layer], c->v_cache[layer], od, 1u, n_rows, pos_0, 0u,
                                     g->n_head_q, g->n_head_kv, g->head_dim, scale, c->stream);
    }
    if (st == LFM_ATTN_OK)
        st = st_of(hipMemcpyAsync(h + in_bytes, od, (size_t)n_rows * qrow * sizeof(float), hipMemcpyDeviceToHost,
                                  c->stream));
    if (st == LFM_ATTN_OK) st = st_of(hipStreamSynchronize(c->stream));
    if (st == LFM_ATTN_OK) memcpy(out, h + in_bytes, (size_t)n_rows * qrow * sizeof(float));
    return st;
}

static int kv_range(lfm_attn_ctx *c, uint32_t layer, uint32_t slot, uint32_t n_slots, size_t *off,
                    size_t *bytes) {
    if (!c || layer >= c->g.n_layers) return LFM_ATTN_E_INVALID;
    if ((uint64_t)slot + n_slots > c->slots[layer]) return LFM_ATTN_E_RANGE;
    const size_t row = (size_t)c->g.n_head_kv * c->g.head_dim;
    *off   = (size_t)slot * row;
    *bytes = (size_t)n_slots * row * sizeof(uint16_t);
    return LFM_ATTN_OK;
}

int lfm_attn_ctx_kv_export(lfm_attn_ctx *c, uint32_t layer, uint32_t slot, uint32_t n_slots,
                           uint16_t *k_host, uint16_t *v_host) {
    size_t off = 0, bytes = 0;
    int st = kv_range(c, layer, slot, n_slots, &off, &bytes);
    if (st != LFM_ATTN_OK) return st;
    if (k_host) st = st_of(hipMemcpyAsync(k_host, c->k_cache[layer] + off, bytes, hipMemcpyDeviceToHost, c->stream));
    if (st == LFM_ATTN_OK && v_host)
        st = st_of(hipMemcpyAsync(v_host, c->v_cache[layer] + off, bytes, hipMemcpyDeviceToHost, c->stream));
    if (st == LFM_ATTN_OK) st = st_of(hipStreamSynchronize(c->stream));
    return st;
}

int lfm_attn_ctx_kv_import(lfm_attn_ctx *c, uint32_t layer, uint32_t slot, uint32_t n_slots,
                           const uint16_t *k_host, const uint16_t *v_host) {
    size_t off = 0, bytes = 0;
    int st = kv_range(c, layer, slot, n_slots, &off, &bytes);
    if (st != LFM_ATTN_OK) return st;
    if (k_host) st = st_of(hipMemcpyAsync(c->k_cache[layer] + off, k_host, bytes, hipMemcpyHostToDevice, c->stream));
    if (st == LFM_ATTN_OK && v_host)
        st = st_of(hipMemcpyAsync(c->v_cache[layer] + off, v_host, bytes, hipMemcpyHostToDevice, c->stream));
    if (st == LFM_ATTN_OK) st = st_of(hipStreamSynchronize(c->stream));
    return st;
}

int lfm_attn_ctx_kv_device(lfm_attn_ctx *c, uint32_t layer, uint16_t **k_dev, uint16_t **v_dev,
                           uint32_t *n_slots) {
    if (!c || layer >= c->g.n_layers) return LFM_ATTN_E_INVALID;
    if (k_dev) *k_dev = c->k_cache[layer];
    if (v_dev) *v_dev = c->v_cache[layer];
    if (n_slots) *n_slots = c->slots[layer];
    return LFM_ATTN_OK;
}

/* Attention-sink eviction over the context's layers: src/lfm2_api.c:871-891
 * calls lfm3_kv_cache_shift_sinks for LFM3 and lfm2_kv_cache_shift_sinks for
 * LFM2 with head_dim 64; the device entry points carry both. */
int lfm_attn_ctx_shift_sinks(lfm_attn_ctx *c, uint32_t *inout_pos, uint32_t n_sink, uint32_t n_discard) {
    if (!c || !inout_pos) return LFM_ATTN_E_INVALID;
    const lfm_attn_geom *g = &c->g;
    const uint32_t L = g->n_layers;
    uint32_t *nkv = (uint32_t *)malloc(L * sizeof(uint32_t));
    uint8_t *kind = (uint8_t *)malloc(L);
    if (!nkv || !kind) {
        free(nkv);
        free(kind);
        return LFM_ATTN_E_NOMEM;
    }
    for (uint32_t l = 0; l < L; ++l) {
        nkv[l]  = g->n_head_kv;
        kind[l] = c->is_swa[l] ? 2u : 1u;
    }
    int st;
    if (!g->lfm3) {
        st = lfm_hip_kv_cache_shift_sinks(c->k_cache, c->v_cache, L, nkv, g->head_dim, c->cos_shift,
                                          c->sin_shift, g->max_seq, inout_pos, n_sink, n_discard,
                                          c->stream);
    } else {
        const float *cs = c->cos_swa ? c->cos_swa : c->cos_full;
        const float *ss = c->sin_swa ? c->sin_swa : c->sin_full;
        st = lfm_hip_lfm3_kv_cache_shift_sinks(c->k_cache, c->v_cache, L, nkv, kind, g->head_dim,
                                               c->cos_full, c->sin_full, g->max_seq, cs, ss, g->max_seq,
                                               g->sliding_window, g->swa_cap, inout_pos, n_sink,
                                               n_discard, c->stream);
    }
    free(nkv);
    free(kind);
    if (st == LFM_ATTN_OK) st = st_of(hipStreamSynchronize(c->stream));
    return st;
}

/* ==== checkpoint SWA ring slab (tools/lfm2_moe_checkpoint.c:472-560) ========== */
int lfm_attn_ctx_swa_slab_bytes(const lfm_attn_ctx *c, size_t *bytes) {
    if (!c || !bytes) return LFM_ATTN_E_INVALID;
    const size_t row = (size_t)c->g.n_head_kv * c->g.head_dim * sizeof(uint16_t);
    size_t b         = 0;
    for (uint32_t l = 0; l < c->g.n_layers; ++l)
        if (c->is_swa[l]) b += 2u * (size_t)c->slots[l] * row;
    *bytes = b;
    return LFM_ATTN_OK;
}

static int swa_slab_copy(lfm_attn_ctx *c, uint8_t *slab, const uint8_t *src_slab) {
    const size_t row = (size_t)c->g.n_head_kv * c->g.head_dim * sizeof(uint16_t);
    size_t off       = 0;
    int st           = LFM_ATTN_OK;
    for (uint32_t l = 0; l < c->g.n_layers && st == LFM_ATTN_OK; ++l) {
        if (!c->is_swa[l]) continue;
        const size_t ring = (size_t)c->slots[l] * row;
        if (slab) {
            st = st_of(hipMemcpyAsync(slab + off, c->k_cache[l], ring, hipMemcpyDefault, c->stream));
            if (st == LFM_ATTN_OK)
                st = st_of(hipMemcpyAsync(slab + off + ring, c->v_cache[l], ring, hipMemcpyDefault, c->stream));
        } else {
            st = st_of(hipMemcpyAsync(c->k_cache[l], src_slab + off, ring, hipMemcpyDefault, c->stream));
            if (st == LFM_ATTN_OK)
                st = st_of(hipMemcpyAsync(c->v_cache[l], src_slab + off + ring, ring, hipMemcpyDefault, c->stream));
        }
        off += 2u * ring;
    }
    if (st == LFM_ATTN_OK) st = st_of(hipStreamSynchronize(c->stream));
    return st;
}

int lfm_attn_ctx_swa_slab_save(lfm_attn_ctx *c, void *slab) {
    if (!c || !slab) return LFM_ATTN_E_INVALID;
    return swa_slab_copy(c, (uint8_t *)slab, NULL);
}

int lfm_attn_ctx_swa_slab_restore(lfm_attn_ctx *c, const void *slab) {
    if (!c || !slab) return LFM_ATTN_E_INVALID;
    return swa_slab_copy(c, NULL, (const uint8_t *)slab);
}

/* ==== prompt cache files (.lfmcache v1) ======================================
 * Layout and rules of tools/lfm2_sys_cache.c:354-799 (header struct :368-380,
 * FNV-1a :382-389, save :504-627, load :650-797). */
#define LFM_CACHE_MAGIC   0x4350324D464C3130ULL /* "01LFM2PC" little-endian */
#define LFM_CACHE_VERSION 1u
#define FNV_OFFSET        14695981039346656037ULL

typedef struct {
    uint64_t magic;
    uint32_t version;
    uint32_t n_tokens;
    uint64_t model_fingerprint;
    uint32_t n_layers;
    uint32_t n_embd;
    uint32_t n_head_q;
    uint32_t shortconv_l_cache;
    uint64_t total_payload_bytes;
    uint8_t reserved[16];
} cache_header;
_Static_assert(sizeof(cache_header) == 64, "cache header is 64 bytes");

/* Per-layer sizes shared by save and load. */
typedef struct {
    uint32_t hist_len, swa_win, cap;
    size_t conv_bytes;
} cache_dims;

static int cache_check(const lfm_attn_ctx *c, const lfm_attn_cache_model *m, cache_dims *d) {
    if (!m || !m->ctx_layer || m->n_model_layers == 0u || m->n_embd == 0u) return LFM_ATTN_E_INVALID;
    for (uint32_t l = 0; l < m->n_model_layers; ++l)
        if (m->ctx_layer[l] >= (int32_t)c->g.n_layers || m->ctx_layer[l] < -1) return LFM_ATTN_E_INVALID;
    d->hist_len   = m->shortconv_l_cache > 1u ? m->shortconv_l_cache - 1u : 2u;
    d->swa_win    = c->g.sliding_window ? c->g.sliding_window : 256u;
    d->cap        = c->g.swa_cap ? c->g.swa_cap : d->swa_win + 8u;
    d->conv_bytes = (size_t)d->hist_len * m->n_embd * sizeof(float);
    return LFM_ATTN_OK;
}

/* Bytes of one attention layer's rows for n positions: K then V. */
static size_t cache_kv_rows(const lfm_attn_ctx *c, uint32_t layer, uint32_t n, const cache_dims *d) {
    const uint32_t rows = c->is_swa[layer] ? (n < d->swa_win ? n : d->swa_win) : n;
    return (size_t)rows * c->g.n_head_kv * c->g.head_dim * sizeof(uint16_t);
}

/* Pinned host buffer for a whole file and a device buffer for its payload. */
static int file_buffers(lfm_attn_ctx *c, size_t host_bytes, size_t dev_bytes) {
    int st = LFM_ATTN_OK;
    if (c->file_host_bytes < host_bytes) {
        if (c->file_host) (void)hipHostFree(c->file_host);
        c->file_host       = NULL;
        c->file_host_bytes = 0;
        st = st_of(hipHostMalloc((void **)&c->file_host, host_bytes, hipHostMallocDefault));
        if (st != LFM_ATTN_OK) return st;
        c->file_host_bytes = host_bytes;
    }
    if (c->file_dev_bytes < dev_bytes) {
        (void)hipFree(c->file_dev);
        c->file_dev       = NULL;
        c->file_dev_bytes = 0;
        st = st_of(hipMalloc((void **)&c->file_dev, dev_bytes));
        if (st != LFM_ATTN_OK) return st;
        c->file_dev_bytes = dev_bytes;
    }
    return st;
}

/* Device-to-device copies of positions [t0, t1) of a layer between its
 * caches and position-ordered K rows at k_rows, V rows at v_rows; ring
 * layers map position t to slot t % cap, in at most two contiguous runs. */
static int cache_rows_d2d(lfm_attn_ctx *c, uint32_t layer, uint32_t t0, uint32_t t1, unsigned char *k_rows,
                          unsigned char *v_rows, const cache_dims *d, int to_cache) {
    const size_t row = (size_t)c->g.n_head_kv * c->g.head_dim * sizeof(uint16_t);
    int st           = LFM_ATTN_OK;
    for (uint32_t t = t0; t < t1 && st == LFM_ATTN_OK;) {
        uint32_t slot = t, n = t1 - t;
        if (c->is_swa[layer]) {
            slot = t % d->cap;
            if (n > d->cap - slot) n = d->cap - slot;
        }
        const size_t o = (size_t)(t - t0) * row, bytes = (size_t)n * row;
        unsigned char *kc = (unsigned char *)c->k_cache[layer] + (size_t)slot * row;
        unsigned char *vc = (unsigned char *)c->v_cache[layer] + (size_t)slot * row;
        st = st_of(hipMemcpyAsync(to_cache ? kc : k_rows + o, to_cache ? k_rows + o : kc, bytes,
                                  hipMemcpyDeviceToDevice, c->stream));
        if (st == LFM_ATTN_OK)
            st = st_of(hipMemcpyAsync(to_cache ? vc : v_rows + o, to_cache ? v_rows + o : vc, bytes,
                                      hipMemcpyDeviceToDevice, c->stream));
        t += n;
    }
    return st;
}

/* Payload bytes of an n-token file. */
static size_t cache_payload(const lfm_attn_ctx *c, const lfm_attn_cache_model *m, uint32_t n, const cache_dims *d) {
    size_t total = (size_t)n * sizeof(uint32_t);
    for (uint32_t l = 0; l < m->n_model_layers; ++l)
        total += m->ctx_layer[l] < 0 ? d->conv_bytes : 2u * cache_kv_rows(c, (uint32_t)m->ctx_layer[l], n, d);
    return total;
}

/* Save: the payload is assembled in device memory in file order (token ids
 * and ShortConv states uploaded, KV rows copied from the caches), hashed
 * there (lfm_hip_fnv1a64), copied out once and written with the header and
 * checksum in one write. */
int lfm_attn_ctx_cache_save(lfm_attn_ctx *c, const char *path, const lfm_attn_cache_model *m,
                            const uint32_t *tokens, uint32_t n_tokens, float *const *conv_states,
                            const uint32_t *conv_ring_heads) {
    if (!c || !path || !tokens || n_tokens == 0u) return LFM_ATTN_E_INVALID;
    cache_dims d;
    int st = cache_check(c, m, &d);
    if (st != LFM_ATTN_OK) return st;
    if (n_tokens > c->g.max_seq) return LFM_ATTN_E_RANGE;
    for (uint32_t l = 0; l < m->n_model_layers; ++l)
        if (m->ctx_layer[l] < 0 && (!conv_states || !conv_states[l])) return LFM_ATTN_E_INVALID;
    char tmp[4096];
    if (snprintf(tmp, sizeof tmp, "%s.tmp.%d", path, (int)getpid()) >= (int)sizeof tmp) return LFM_ATTN_E_INVALID;
    const size_t payload = cache_payload(c, m, n_tokens, &d);
    st = file_buffers(c, sizeof(cache_header) + payload + sizeof(uint64_t), align256(payload));
    if (st != LFM_ATTN_OK) return st;
    unsigned char *hp = c->file_host + sizeof(cache_header), *dp = c->file_dev;

    size_t off = (size_t)n_tokens * sizeof(uint32_t);
    memcpy(hp, tokens, off);
    st = st_of(hipMemcpyAsync(dp, hp, off, hipMemcpyHostToDevice, c->stream));
    for (uint32_t l = 0; l < m->n_model_layers && st == LFM_ATTN_OK; ++l) {
        if (m->ctx_layer[l] < 0) {
            const float *src = conv_states[l];
            for (uint32_t sidx = 0; sidx < d.hist_len; ++sidx) {
                const uint32_t slot = conv_ring_heads && d.hist_len > 1u ? (conv_ring_heads[l] + sidx) % d.hist_len
                                                                         : sidx;
                memcpy(hp + off + (size_t)sidx * m->n_embd * sizeof(float), src + (size_t)slot * m->n_embd,
                       (size_t)m->n_embd * sizeof(float));
            }
            st = st_of(hipMemcpyAsync(dp + off, hp + off, d.conv_bytes, hipMemcpyHostToDevice, c->stream));
            off += d.conv_bytes;
        } else {
            const uint32_t layer = (uint32_t)m->ctx_layer[l];
            const size_t b       = cache_kv_rows(c, layer, n_tokens, &d);
            const uint32_t rows  = (uint32_t)(b / ((size_t)c->g.n_head_kv * c->g.head_dim * sizeof(uint16_t)));
            st = cache_rows_d2d(c, layer, n_tokens - rows, n_tokens, dp + off, dp + off + b, &d, 0);
            off += 2u * b;
        }
    }
    uint64_t csum = 0;
    if (st == LFM_ATTN_OK) st = lfm_hip_fnv1a64(dp, payload, FNV_OFFSET, &csum, c->stream);
    if (st == LFM_ATTN_OK) st = st_of(hipMemcpyAsync(hp, dp, payload, hipMemcpyDeviceToHost, c->stream));
    if (st == LFM_ATTN_OK) st = st_of(hipStreamSynchronize(c->stream));
    if (st != LFM_ATTN_OK) return st;

    cache_header h;
    memset(&h, 0, sizeof h);
    h.magic               = LFM_CACHE_MAGIC;
    h.version             = LFM_CACHE_VERSION;
    h.n_tokens            = n_tokens;
    h.model_fingerprint   = m->model_fingerprint;
    h.n_layers            = m->n_model_layers;
    h.n_embd              = m->n_embd;
    h.n_head_q            = m->n_head_q;
    h.shortconv_l_cache   = m->shortconv_l_cache;
    h.total_payload_bytes = payload;
    memcpy(c->file_host, &h, sizeof h);
    memcpy(hp + payload, &csum, sizeof csum);

    const size_t total = sizeof h + payload + sizeof csum;
    FILE *f            = fopen(tmp, "wb");
    if (!f) return LFM_ATTN_E_IO;
    st = fwrite(c->file_host, 1, total, f) == total && fflush(f) == 0 ? LFM_ATTN_OK : LFM_ATTN_E_IO;
    if (st == LFM_ATTN_OK) (void)fsync(fileno(f));
    if (fclose(f) != 0) st = LFM_ATTN_E_IO;
    if (st == LFM_ATTN_OK && rename(tmp, path) != 0) st = LFM_ATTN_E_IO;
    if (st != LFM_ATTN_OK) (void)unlink(tmp);
    return st;
}

/* Load: header checks, the whole payload read into pinned memory, the token
 * prefix compared, the payload uploaded and its checksum verified on the
 * device; only then are the states and caches written (caches by
 * device-to-device copies from the uploaded payload). */
int lfm_attn_ctx_cache_load_prefix(lfm_attn_ctx *c, const char *path, const lfm_attn_cache_model *m,
                                   const uint32_t *prompt, uint32_t n_prompt, float *const *conv_states,
                                   uint32_t *out_conv_heads, uint32_t *matched_pos) {
    if (!matched_pos) return LFM_ATTN_E_INVALID;
    *matched_pos = 0;
    if (!c || !path || !prompt) return LFM_ATTN_E_INVALID;
    cache_dims d;
    int st = cache_check(c, m, &d);
    if (st != LFM_ATTN_OK) return st;
    FILE *f = fopen(path, "rb");
    if (!f) return LFM_ATTN_OK;
    cache_header h;
    if (fread(&h, sizeof h, 1, f) != 1 || h.magic != LFM_CACHE_MAGIC || h.version != LFM_CACHE_VERSION ||
        h.model_fingerprint != m->model_fingerprint || h.n_layers != m->n_model_layers ||
        h.n_embd != m->n_embd || h.n_tokens == 0u || h.n_tokens > n_prompt || h.n_tokens > c->g.max_seq) {
        fclose(f);
        return LFM_ATTN_OK;
    }
    const uint32_t n      = h.n_tokens;
    const size_t payload  = cache_payload(c, m, n, &d);
    st = file_buffers(c, sizeof h + payload + sizeof(uint64_t), align256(payload));
    if (st != LFM_ATTN_OK) {
        fclose(f);
        return st;
    }
    unsigned char *hp = c->file_host + sizeof h, *dp = c->file_dev;
    const int whole   = fread(hp, 1, payload + sizeof(uint64_t), f) == payload + sizeof(uint64_t);
    fclose(f);
    if (!whole || memcmp(hp, prompt, (size_t)n * sizeof(uint32_t)) != 0) return LFM_ATTN_OK;
    uint64_t stored = 0, csum = 0;
    memcpy(&stored, hp + payload, sizeof stored);
    st = st_of(hipMemcpyAsync(dp, hp, payload, hipMemcpyHostToDevice, c->stream));
    if (st == LFM_ATTN_OK) st = lfm_hip_fnv1a64(dp, payload, FNV_OFFSET, &csum, c->stream);
    if (st != LFM_ATTN_OK || csum != stored) return st;

    size_t off = (size_t)n * sizeof(uint32_t);
    for (uint32_t l = 0; l < m->n_model_layers && st == LFM_ATTN_OK; ++l) {
        if (m->ctx_layer[l] < 0) {
            if (conv_states && conv_states[l]) {
                memcpy(conv_states[l], hp + off, d.conv_bytes);
                if (out_conv_heads) out_conv_heads[l] = 0u;
            }
            off += d.conv_bytes;
        } else {
            const uint32_t layer = (uint32_t)m->ctx_layer[l];
            const size_t b       = cache_kv_rows(c, layer, n, &d);
            const uint32_t rows  = (uint32_t)(b / ((size_t)c->g.n_head_kv * c->g.head_dim * sizeof(uint16_t)));
            st = cache_rows_d2d(c, layer, n - rows, n, dp + off, dp + off + b, &d, 1);
            off += 2u * b;
        }
    }
    if (st == LFM_ATTN_OK) st = st_of(hipStreamSynchronize(c->stream));
    if (st == LFM_ATTN_OK) *matched_pos = n;
    return st;
}
