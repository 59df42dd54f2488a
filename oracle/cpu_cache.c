/*
 * oracle/cpu_cache.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Host restatement of the engine's KV persistence formats, the checker for
 * the context's .lfmcache writer/loader and its checkpoint slab:
 *   - .lfmcache v1 prompt cache: tools/lfm2_sys_cache.c:354-799
 *     (header :368-380, FNV-1a :382-389, fingerprint :392-422,
 *     save :504-627, prefix load :650-797);
 *   - LFM2Checkpoint SWA ring slab: tools/lfm2_moe_checkpoint.c:399-560.
 * Layer kinds: 0 ShortConv, 1 full attention, 2 sliding-window attention.
 */
#define _POSIX_C_SOURCE 200809L
#include "cpu_attn.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define PC_MAGIC   0x4350324D464C3130ULL
#define PC_VERSION 1u
#define FNV_BASIS  14695981039346656037ULL
#define FNV_MULT   1099511628211ULL

/* tools/lfm2_sys_cache.c:382-389 */
uint64_t orc_fnv1a(uint64_t h, const void *data, size_t len) {
    const uint8_t *b = (const uint8_t *)data;
    for (size_t i = 0; i < len; ++i) h = (h ^ b[i]) * FNV_MULT;
    return h;
}

/* tools/lfm2_sys_cache.c:394-422 without the tensor list (names, types and
 * dims of the model file's tensors, hashed last; the engine supplies them). */
uint64_t orc_model_fingerprint(const char *arch, uint32_t n_layers, uint32_t n_embd, uint32_t n_vocab,
                               uint32_t n_head_q, uint32_t l_cache, const uint32_t *n_head_kv, int is_lfm3,
                               uint32_t head_dim, uint32_t sliding_window, const uint8_t *is_swa) {
    uint64_t h = orc_fnv1a(FNV_BASIS, arch, strlen(arch));
    h          = orc_fnv1a(h, &n_layers, 4);
    h          = orc_fnv1a(h, &n_embd, 4);
    h          = orc_fnv1a(h, &n_vocab, 4);
    h          = orc_fnv1a(h, &n_head_q, 4);
    h          = orc_fnv1a(h, &l_cache, 4);
    h          = orc_fnv1a(h, n_head_kv, 4u * (size_t)n_layers);
    if (is_lfm3) {
        h = orc_fnv1a(h, &head_dim, 4);
        h = orc_fnv1a(h, &sliding_window, 4);
        h = orc_fnv1a(h, is_swa, n_layers); /* one byte per layer (C bool) */
    }
    return h;
}

typedef struct {
    uint32_t hist, win, cap;
    size_t conv_bytes;
} pc_dims;

static pc_dims pc_dims_of(uint32_t n_embd, uint32_t l_cache, uint32_t sliding_window, uint32_t swa_cap) {
    pc_dims d;
    d.hist       = l_cache > 1u ? l_cache - 1u : 2u;
    d.win        = sliding_window ? sliding_window : 256u;
    d.cap        = swa_cap ? swa_cap : d.win + 8u;
    d.conv_bytes = (size_t)d.hist * n_embd * sizeof(float);
    return d;
}

/* positions a layer keeps: all n (full), the last min(n, win) (SWA) */
static uint32_t pc_first_pos(uint8_t kind, uint32_t n, const pc_dims *d) {
    return kind == 2u && n > d->win ? n - d->win : 0u;
}

/* lfm2_prompt_cache_save_ex (tools/lfm2_sys_cache.c:504-627); 1 on success */
int orc_prompt_cache_save(const char *path, uint64_t fingerprint, uint32_t n_layers, const uint32_t *n_head_kv,
                          const uint8_t *layer_kind, uint32_t head_dim, uint32_t n_embd, uint32_t n_head_q,
                          uint32_t l_cache, uint32_t sliding_window, const uint32_t *tokens, uint32_t n_tokens,
                          float *const *conv, const uint32_t *conv_heads, uint16_t *const *k, uint16_t *const *v,
                          uint32_t swa_cap) {
    if (!path || !tokens || n_tokens == 0u) return 0;
    const pc_dims d = pc_dims_of(n_embd, l_cache, sliding_window, swa_cap);
    uint8_t hdr[64];
    memset(hdr, 0, sizeof hdr);
    uint64_t payload = 4ull * n_tokens;
    for (uint32_t l = 0; l < n_layers; ++l)
        payload += layer_kind[l] == 0u ? d.conv_bytes
                                       : 4ull * (n_tokens - pc_first_pos(layer_kind[l], n_tokens, &d)) *
                                             n_head_kv[l] * head_dim;
    const uint64_t magic = PC_MAGIC;
    const uint32_t u32s[2] = {PC_VERSION, n_tokens}, u32b[4] = {n_layers, n_embd, n_head_q, l_cache};
    memcpy(hdr, &magic, 8);
    memcpy(hdr + 8, u32s, 8);
    memcpy(hdr + 16, &fingerprint, 8);
    memcpy(hdr + 24, u32b, 16);
    memcpy(hdr + 40, &payload, 8);

    char tmp[1024];
    snprintf(tmp, sizeof tmp, "%s.tmp.%d", path, (int)getpid());
    FILE *f = fopen(tmp, "wb");
    if (!f) return 0;
    int ok        = fwrite(hdr, 1, 64, f) == 64;
    uint64_t csum = FNV_BASIS;
#define EMIT(p, n)                                                    \
    do {                                                              \
        if (ok && (n) > 0) {                                          \
            ok   = fwrite((p), 1, (n), f) == (size_t)(n);             \
            csum = orc_fnv1a(csum, (p), (n));                         \
        }                                                             \
    } while (0)
    EMIT(tokens, 4u * (size_t)n_tokens);
    for (uint32_t l = 0; l < n_layers && ok; ++l) {
        if (layer_kind[l] == 0u) {
            /* ring slot (head + s) % hist holds the s-th oldest row */
            for (uint32_t s = 0; s < d.hist; ++s) {
                const uint32_t slot = conv_heads && d.hist > 1u ? (conv_heads[l] + s) % d.hist : s;
                EMIT(conv[l] + (size_t)slot * n_embd, (size_t)n_embd * sizeof(float));
            }
            continue;
        }
        const size_t row   = (size_t)n_head_kv[l] * head_dim;
        const uint32_t t0  = pc_first_pos(layer_kind[l], n_tokens, &d);
        uint16_t *const *c = k;
        for (int pass = 0; pass < 2; ++pass, c = v)
            for (uint32_t t = t0; t < n_tokens; ++t) {
                const uint32_t slot = layer_kind[l] == 2u ? t % d.cap : t;
                EMIT(c[l] + (size_t)slot * row, row * sizeof(uint16_t));
            }
    }
#undef EMIT
    if (ok) ok = fwrite(&csum, 8, 1, f) == 1;
    if (fclose(f) != 0) ok = 0;
    if (ok && rename(tmp, path) != 0) ok = 0;
    if (!ok) unlink(tmp);
    return ok;
}

/* lfm2_prompt_cache_try_load_prefix_ex (tools/lfm2_sys_cache.c:650-797):
 * streams the payload into the buffers as it verifies, as the reference does;
 * returns the matched position, 0 when the file does not apply. */
uint32_t orc_prompt_cache_load(const char *path, uint64_t fingerprint, uint32_t n_layers,
                               const uint32_t *n_head_kv, const uint8_t *layer_kind, uint32_t head_dim,
                               uint32_t n_embd, uint32_t n_head_q, uint32_t l_cache, uint32_t sliding_window,
                               const uint32_t *prompt, uint32_t n_prompt, uint32_t max_seq, float *const *conv,
                               uint32_t *conv_heads, uint16_t *const *k, uint16_t *const *v, uint32_t swa_cap) {
    (void)n_head_q;
    FILE *f = path ? fopen(path, "rb") : NULL;
    if (!f || !prompt) {
        if (f) fclose(f);
        return 0;
    }
    uint8_t hdr[64];
    uint64_t magic = 0, fp = 0;
    uint32_t ver = 0, n = 0, hl = 0, he = 0;
    int ok = fread(hdr, 1, 64, f) == 64;
    memcpy(&magic, hdr, 8);
    memcpy(&ver, hdr + 8, 4);
    memcpy(&n, hdr + 12, 4);
    memcpy(&fp, hdr + 16, 8);
    memcpy(&hl, hdr + 24, 4);
    memcpy(&he, hdr + 28, 4);
    ok = ok && magic == PC_MAGIC && ver == PC_VERSION && fp == fingerprint && hl == n_layers && he == n_embd &&
         n != 0u && n <= n_prompt && n <= max_seq;
    uint64_t csum = FNV_BASIS;
#define TAKE(p, len)                                                  \
    do {                                                              \
        if (ok) {                                                     \
            ok = fread((p), 1, (len), f) == (size_t)(len);            \
            if (ok) csum = orc_fnv1a(csum, (p), (len));               \
        }                                                             \
    } while (0)
    uint32_t *ids = ok ? (uint32_t *)malloc(4u * (size_t)n) : NULL;
    if (ok && !ids) ok = 0;
    TAKE(ids, 4u * (size_t)n);
    if (ok) ok = memcmp(ids, prompt, 4u * (size_t)n) == 0;
    free(ids);
    const pc_dims d = pc_dims_of(n_embd, l_cache, sliding_window, swa_cap);
    uint8_t *sink   = (uint8_t *)malloc(d.conv_bytes + (size_t)65536 * 4u);
    if (!sink) ok = 0;
    for (uint32_t l = 0; l < n_layers && ok; ++l) {
        if (layer_kind[l] == 0u) {
            const int keep = conv && conv[l];
            TAKE(keep ? (void *)conv[l] : (void *)sink, d.conv_bytes);
            if (ok && keep && conv_heads) conv_heads[l] = 0u;
            continue;
        }
        const size_t row   = (size_t)n_head_kv[l] * head_dim * sizeof(uint16_t);
        const uint32_t t0  = pc_first_pos(layer_kind[l], n, &d);
        const int keep     = k && v && k[l] && v[l];
        uint16_t *const *c = k;
        for (int pass = 0; pass < 2; ++pass, c = v)
            for (uint32_t t = t0; t < n && ok; ++t) {
                const uint32_t slot = layer_kind[l] == 2u ? t % d.cap : t;
                if (keep) TAKE((uint8_t *)c[l] + (size_t)slot * row, row);
                else
                    for (size_t r = 0; r < row && ok; r += 65536u * 4u) {
                        const size_t chunk = row - r < 65536u * 4u ? row - r : 65536u * 4u;
                        TAKE(sink, chunk);
                    }
            }
    }
#undef TAKE
    free(sink);
    uint64_t stored = 0;
    if (ok) ok = fread(&stored, 8, 1, f) == 1 && stored == csum;
    fclose(f);
    return ok ? n : 0u;
}

/* LFM2Checkpoint SWA slab (tools/lfm2_moe_checkpoint.c:472-560): whole
 * K ring then V ring of every SWA layer in order; restore != 0 copies back.
 * Returns the slab length in uint16 elements. */
size_t orc_checkpoint_swa_slab(uint16_t *slab, uint32_t n_layers, const uint32_t *n_head_kv,
                               const uint8_t *layer_kind, uint32_t head_dim, uint32_t swa_cap,
                               uint16_t *const *k, uint16_t *const *v, int restore) {
    size_t off = 0;
    for (uint32_t l = 0; l < n_layers; ++l) {
        if (layer_kind[l] != 2u) continue;
        const size_t ring = (size_t)swa_cap * n_head_kv[l] * head_dim;
        if (slab) {
            for (int pass = 0; pass < 2; ++pass) {
                uint16_t *cache = pass ? v[l] : k[l];
                uint16_t *part  = slab + off + (size_t)pass * ring;
                memcpy(restore ? cache : part, restore ? part : cache, ring * sizeof(uint16_t));
            }
        }
        off += 2u * ring;
    }
    return off;
}
