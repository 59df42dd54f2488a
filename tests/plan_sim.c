/*
 * plan_sim.c -- CPU simulation of the balanced split-KV plan of
 * k_splitkv_bal / k_merge_bal, built on the same header the kernels use
 * (laii_amd/csrc/splitkv_plan.h).  Test infrastructure: compiled by
 * tests/test_splitkv_plan.py with gcc and called through ctypes.
 *
 * plan_check() runs every launched workgroup's walk exactly as the kernel
 * does (the per-lane prefix search of find_seq is emulated in 64-lane
 * batches), records every write -- a direct output or a partial slot -- and
 * then runs the merge's slot range for every (sequence, KV head).  It checks:
 *   - every key of [t_start(pos0), pos0 + n_rows - 1] of every (sequence, KV
 *     head) is covered by exactly one segment (tools/lfm3_engine.c:862-873);
 *   - partial slots are unique per KV head and below the workspace's slot
 *     count (lfm_bal_n_slots);
 *   - a unit written directly has exactly one segment, and the merge leaves it
 *     alone; otherwise the merge reads exactly the slots written for it.
 * Returns 0, or a negative code with a message in msg.
 *
 * mutant != 0 plants a mistake in the simulated plan (1: the partial slot
 * drops the group term; 2: the merge's last workgroup is off by one; 3: a
 * segment's last key is not clipped to the rows' last key), which the checks
 * must reject.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "splitkv_plan.h"

typedef struct {
    uint32_t kb, ke;
    int64_t slot; /* -1: direct output */
} seg_rec;

/* The sequence holding tile t and its first tile, as find_seq computes them
 * on the device: 64 sequences per pass, an inclusive scan of n_groups *
 * tiles(s) over the lanes, the first lane whose running total exceeds t. */
static void find_seq_wave(const lfm_bal_cfg *c, const uint32_t *pos0, uint64_t t, uint32_t *s_out,
                          uint64_t *first_out) {
    uint64_t base = 0;
    for (uint32_t b = 0;; b += 64u) {
        uint32_t incl[64], x[64], run = 0;
        for (uint32_t l = 0; l < 64u; ++l) {
            const uint32_t s = b + l;
            x[l]             = s < c->n_seq ? lfm_bal_seq_tiles(c, pos0[s]) * c->n_groups : 0u;
            run += x[l];
            incl[l] = run;
        }
        const uint32_t tot = incl[63];
        if (t < base + tot || b + 64u >= c->n_seq) {
            int l = 0;
            for (int k = 0; k < 64; ++k)
                if (base + incl[k] > t) { l = k; break; }
            *s_out     = b + (uint32_t)l;
            *first_out = base + incl[l] - x[l];
            return;
        }
        base += tot;
    }
}

#define FAIL(code, ...)                                  \
    do {                                                 \
        snprintf(msg, msg_len, __VA_ARGS__);             \
        rc = (code);                                     \
        goto done;                                       \
    } while (0)

/* W: KV heads per workgroup (waves); ncols: query columns per KV head. */
int plan_check(uint32_t n_seq, const uint32_t *pos0, uint32_t n_rows, uint32_t n_head_kv, uint32_t W,
               uint32_t window, uint32_t cap, uint32_t ncols, uint32_t n_res, uint32_t target_waves,
               uint32_t min_tiles, uint32_t keys, int mutant, uint32_t *out_G, uint32_t *out_wg, char *msg,
               size_t msg_len) {
    int rc = 0;
    lfm_bal_cfg c;
    memset(&c, 0, sizeof c);
    c.n_seq        = n_seq;
    c.n_rows       = n_rows;
    c.n_head_kv    = n_head_kv;
    c.n_groups     = (n_head_kv + W - 1u) / W;
    c.window       = window;
    c.cap          = cap;
    c.min_tiles    = min_tiles;
    c.n_res        = n_res;
    c.target_waves = target_waves;
    c.n_wg         = lfm_bal_launch_wgs(&c, keys);
    (void)ncols;

    /* tile_plan */
    uint64_t T64 = 0;
    int uniform  = 1;
    const uint32_t t0 = lfm_bal_seq_tiles(&c, pos0[0]);
    for (uint32_t s = 0; s < n_seq; ++s) {
        const uint32_t x = lfm_bal_seq_tiles(&c, pos0[s]);
        T64 += x;
        if (x != t0) uniform = 0;
    }
    if (T64 > 0xFFFFFFFFull) { snprintf(msg, msg_len, "T overflows"); return -9; }
    const uint32_t T = (uint32_t)T64;
    const uint32_t G = lfm_bal_plan_wgs(&c, T, uniform);
    *out_G           = G;
    *out_wg          = c.n_wg;
    const uint64_t n_slots = lfm_bal_n_slots(c.n_wg, c.n_groups, c.n_seq);
    if (G > c.n_wg) { snprintf(msg, msg_len, "G %u > launched %u", G, c.n_wg); return -1; }

    /* per (s, kvh): recorded segments */
    const size_t pairs = (size_t)n_seq * n_head_kv;
    size_t cap_rec     = 16;
    seg_rec **rec      = calloc(pairs, sizeof *rec);
    uint32_t *nrec     = calloc(pairs, sizeof *nrec);
    uint32_t *caprec   = calloc(pairs, sizeof *caprec);
    uint8_t *slot_used = calloc((size_t)n_slots * n_head_kv, 1);
    uint32_t *prefix   = calloc((size_t)n_seq + 2u, sizeof *prefix);
    if (!rec || !nrec || !caprec || !slot_used || !prefix) FAIL(-8, "out of memory");
    (void)cap_rec;

#define RECORD(S, KVH, KB, KE, SLOT)                                                              \
    do {                                                                                          \
        const size_t pr_ = (size_t)(S) * n_head_kv + (KVH);                                       \
        if (nrec[pr_] == caprec[pr_]) {                                                           \
            caprec[pr_] = caprec[pr_] ? 2u * caprec[pr_] : 8u;                                    \
            rec[pr_]    = realloc(rec[pr_], caprec[pr_] * sizeof(seg_rec));                       \
            if (!rec[pr_]) FAIL(-8, "out of memory");                                             \
        }                                                                                         \
        rec[pr_][nrec[pr_]].kb   = (KB);                                                          \
        rec[pr_][nrec[pr_]].ke   = (KE);                                                          \
        rec[pr_][nrec[pr_]].slot = (SLOT);                                                        \
        nrec[pr_]++;                                                                              \
        if ((SLOT) >= 0) {                                                                        \
            if ((uint64_t)(SLOT) >= n_slots) FAIL(-2, "slot %lld >= %llu", (long long)(SLOT),     \
                                                   (unsigned long long)n_slots);                  \
            uint8_t *u_ = &slot_used[(size_t)(SLOT) * n_head_kv + (KVH)];                         \
            if (*u_) FAIL(-3, "slot %lld kvh %u written twice", (long long)(SLOT), (KVH));        \
            *u_ = 1;                                                                              \
        }                                                                                         \
    } while (0)

    /* the kernel's workgroups */
    for (uint32_t wg = 0; wg < c.n_wg; ++wg) {
        if (wg >= G) continue;
        if (uniform) {
            const lfm_bal_useg u = lfm_bal_uniform_segment(&c, wg, G, T / n_seq);
            if (u.n == 0u) FAIL(-4, "uniform plan with no workgroup per unit");
            for (uint32_t w = 0; w < W; ++w) {
                const uint32_t kvh = u.grp * W + w;
                if (kvh >= n_head_kv) continue;
                uint32_t kb, ke;
                lfm_bal_seg_keys(&c, pos0[u.s], u.a, u.b, &kb, &ke);
                RECORD(u.s, kvh, kb, ke, u.n == 1u ? (int64_t)-1 : (int64_t)u.slot);
            }
            continue;
        }
        const uint64_t N = (uint64_t)T * c.n_groups;
        uint64_t t, t1;
        lfm_bal_wg_tiles(wg, N, G, &t, &t1);
        uint32_t s;
        uint64_t first;
        find_seq_wave(&c, pos0, t, &s, &first);
        while (t < t1) {
            if (s >= n_seq) FAIL(-5, "walk past the last sequence (wg %u)", wg);
            const uint32_t tiles = lfm_bal_seq_tiles(&c, pos0[s]);
            const lfm_bal_seg sg = lfm_bal_segment(t, t1, first, tiles);
            if (sg.grp >= c.n_groups) FAIL(-5, "group %u out of range (wg %u)", sg.grp, wg);
            for (uint32_t w = 0; w < W; ++w) {
                const uint32_t kvh = sg.grp * W + w;
                if (kvh >= n_head_kv) continue;
                uint32_t kb, ke;
                lfm_bal_seg_keys(&c, pos0[s], sg.a, sg.b, &kb, &ke);
                if (mutant == 3) ke = lfm_plan_row(pos0[s], window, cap).t_start + 32u * sg.b;
                const uint64_t slot = mutant == 1 ? (uint64_t)wg + (uint64_t)s * c.n_groups
                                                  : lfm_bal_slot(wg, s, c.n_groups, sg.grp);
                RECORD(s, kvh, kb, ke, sg.whole ? (int64_t)-1 : (int64_t)slot);
            }
            t = sg.end;
            if (t == first + (uint64_t)tiles * c.n_groups) {
                first = t;
                ++s;
            }
        }
    }

    /* tile prefix (workgroup 0) */
    {
        uint32_t base = 0;
        for (uint32_t s = 0; s < n_seq; ++s) {
            prefix[s] = base;
            base += lfm_bal_seq_tiles(&c, pos0[s]);
        }
        prefix[n_seq]      = base;
        prefix[n_seq + 1u] = G;
    }

    /* coverage and the merge's reads */
    for (uint32_t s = 0; s < n_seq; ++s) {
        const uint32_t lo   = lfm_plan_row(pos0[s], window, cap).t_start;
        const uint32_t last = pos0[s] + n_rows - 1u;
        const uint32_t grp_tiles = prefix[s + 1u] - prefix[s];
        for (uint32_t kvh = 0; kvh < n_head_kv; ++kvh) {
            const size_t pr = (size_t)s * n_head_kv + kvh;
            const uint32_t n = nrec[pr];
            if (n == 0u) FAIL(-6, "seq %u kvh %u: no segment", s, kvh);
            /* sort by kb (insertion sort; few segments) */
            seg_rec *r = rec[pr];
            for (uint32_t i = 1; i < n; ++i) {
                seg_rec x = r[i];
                uint32_t j = i;
                while (j > 0 && r[j - 1].kb > x.kb) { r[j] = r[j - 1]; --j; }
                r[j] = x;
            }
            if (r[0].kb != lo) FAIL(-6, "seq %u kvh %u: first key %u != %u", s, kvh, r[0].kb, lo);
            for (uint32_t i = 0; i < n; ++i) {
                if (r[i].ke <= r[i].kb) FAIL(-6, "seq %u kvh %u: empty segment [%u,%u)", s, kvh, r[i].kb, r[i].ke);
                if (i + 1 < n && r[i].ke != r[i + 1].kb)
                    FAIL(-6, "seq %u kvh %u: gap/overlap at %u/%u", s, kvh, r[i].ke, r[i + 1].kb);
            }
            if (r[n - 1].ke != last + 1u) FAIL(-6, "seq %u kvh %u: last key %u != %u", s, kvh, r[n - 1].ke, last + 1u);
            const uint32_t grp = kvh / W;
            uint32_t g0, g1;
            lfm_bal_merge_range(prefix[s], grp_tiles, grp, prefix[n_seq], c.n_groups, prefix[n_seq + 1u], &g0, &g1);
            if (mutant == 2 && g1 + 1u < prefix[n_seq + 1u]) ++g1;
            if (g0 == g1) {
                if (n != 1u || r[0].slot != -1)
                    FAIL(-7, "seq %u kvh %u: merge skips a unit of %u segments", s, kvh, n);
                continue;
            }
            if (n != g1 - g0 + 1u) FAIL(-7, "seq %u kvh %u: %u segments, merge reads %u", s, kvh, n, g1 - g0 + 1u);
            for (uint32_t g = g0; g <= g1; ++g) {
                const int64_t slot = (int64_t)lfm_bal_slot(g, s, c.n_groups, grp);
                int found = 0;
                for (uint32_t i = 0; i < n; ++i) found |= r[i].slot == slot;
                if (!found) FAIL(-7, "seq %u kvh %u: merge reads slot %lld never written", s, kvh, (long long)slot);
            }
        }
    }
done:
    if (rec)
        for (size_t i = 0; i < pairs; ++i) free(rec[i]);
    free(rec);
    free(nrec);
    free(caprec);
    free(slot_used);
    free(prefix);
    return rc;
}
