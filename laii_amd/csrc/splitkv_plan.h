/*
 * splitkv_plan.h -- integer plan of the balanced split-KV decode
 * (k_splitkv_bal / k_merge_bal in decode_splitkv.hip).
 *
 * One header, compiled into the kernels (functions are __host__ __device__
 * under hipcc), into the host launch code, and into the CPU plan check of the
 * tests, so the index math the tests prove is the math the device runs.
 *
 * Keys of the batch are cut into 32-key tiles.  The tiles of every
 * (sequence, KV-head group) unit are laid out as one sequence: sequence
 * major, then group, then tile; unit v = s * n_groups + grp holds
 * `tiles(s)` tiles.  Each row of sequence s attends keys
 * [t_start(pos0[s]), pos0[s] + n_rows - 1] (tools/lfm3_engine.c:862-873);
 * the tiles of a unit cover the union of its rows' keys.
 *
 * Ragged batches: workgroup wg of G takes tiles [wg*N/G, (wg+1)*N/G) of the
 * N = T * n_groups tiles (T = sum of tiles(s)), cut at unit boundaries into
 * segments.  Segment (wg, unit v) writes partial slot wg + v: the workgroups
 * meeting unit v are owner(first tile) .. owner(last tile), a run that no
 * other unit's slots overlap, so slots are unique and below G + units.  A
 * unit one workgroup covers whole is written directly (no partial).
 *
 * Uniform batches (every sequence the same tile count): every unit gets
 * n = G / units equal workgroups; workgroup wg takes unit wg / n, share
 * wg % n, slot wg + unit.
 */
#ifndef LFM_SPLITKV_PLAN_H
#define LFM_SPLITKV_PLAN_H

#include <stdint.h>

#include "attn_index.h"

typedef struct {
    uint32_t n_seq;        /* sequences of the batch                           */
    uint32_t n_rows;       /* query rows per sequence                          */
    uint32_t n_head_kv;
    uint32_t n_groups;     /* KV-head groups (one wave per KV head of a group)  */
    uint32_t window, cap;  /* sliding window and ring slots (0: linear cache)  */
    uint32_t n_wg;         /* workgroups launched                              */
    uint32_t min_tiles;    /* fewest tiles per workgroup on a ragged batch     */
    uint32_t n_res;        /* workgroups resident on the device at once        */
    uint32_t target_waves; /* waves over a uniform batch                       */
} lfm_bal_cfg;

/* 32-key tiles covering the keys the rows of a sequence at pos0 attend. */
LFM_IDX_FN uint32_t lfm_bal_seq_tiles(const lfm_bal_cfg *c, uint32_t pos0) {
    const uint32_t lo = lfm_plan_row(pos0, c->window, c->cap).t_start;
    return (pos0 + c->n_rows - 1u - lo + 32u) >> 5;
}

/* Workgroups taking part, for T tiles per group over the batch. */
LFM_IDX_FN uint32_t lfm_bal_plan_wgs(const lfm_bal_cfg *c, uint32_t T, int uniform) {
    const uint64_t N     = (uint64_t)T * c->n_groups;
    const uint32_t units = c->n_seq * c->n_groups;
    uint64_t G;
    if (uniform) {
        /* every unit gets n equal workgroups, about target_waves waves over
         * the batch (one residency round at the launcher's target) */
        const uint32_t tiles = T / c->n_seq;
        uint64_t ct = ((uint64_t)tiles * c->n_seq * c->n_head_kv + c->target_waves - 1u) / c->target_waves;
        if (ct < c->min_tiles) ct = c->min_tiles;
        G = (uint64_t)units * ((tiles + ct - 1u) / ct);
    } else {
        /* one residency round of equal shares */
        G = N / c->min_tiles;
        if (G > c->n_res) G = c->n_res;
    }
    if (G > c->n_wg) G = c->n_wg;
    if (uniform && G >= units) G -= G % units;
    return (uint32_t)(G ? G : 1u);
}

/* Workgroup holding tile t of n_tiles shared by G workgroups. */
LFM_IDX_FN uint32_t lfm_bal_tile_owner(uint64_t t, uint64_t n_tiles, uint32_t G) {
    return (uint32_t)(((t + 1u) * G - 1u) / n_tiles);
}

/* Tiles [*t0, *t1) of workgroup wg. */
LFM_IDX_FN void lfm_bal_wg_tiles(uint32_t wg, uint64_t n_tiles, uint32_t G, uint64_t *t0, uint64_t *t1) {
    *t0 = (uint64_t)wg * n_tiles / G;
    *t1 = (uint64_t)(wg + 1u) * n_tiles / G;
}

/* One segment of a ragged workgroup's walk: its tiles from t (inside the
 * units of sequence s, whose first tile is `first`, `tiles` per unit) up
 * to t1 or the end of the unit. */
typedef struct {
    uint32_t grp;  /* KV-head group of the unit                 */
    uint32_t a, b; /* tiles [a, b) of the unit                  */
    uint64_t end;  /* tile after the segment (the next t)       */
    int whole;     /* the segment is the unit's only one         */
} lfm_bal_seg;

LFM_IDX_FN lfm_bal_seg lfm_bal_segment(uint64_t t, uint64_t t1, uint64_t first, uint32_t tiles) {
    lfm_bal_seg g;
    g.grp             = (uint32_t)((t - first) / tiles);
    const uint64_t u0 = first + (uint64_t)g.grp * tiles; /* the unit's tile 0 */
    g.end             = t1 < u0 + tiles ? t1 : u0 + tiles;
    g.a               = (uint32_t)(t - u0);
    g.b               = (uint32_t)(g.end - u0);
    g.whole           = g.a == 0u && g.b == tiles;
    return g;
}

/* Keys [*kb, *ke) of tiles [a, b) of a sequence at pos0. */
LFM_IDX_FN void lfm_bal_seg_keys(const lfm_bal_cfg *c, uint32_t pos0, uint32_t a, uint32_t b, uint32_t *kb,
                                 uint32_t *ke) {
    const uint32_t lo   = lfm_plan_row(pos0, c->window, c->cap).t_start;
    const uint32_t end  = pos0 + c->n_rows;
    const uint32_t e    = lo + 32u * b;
    *kb = lo + 32u * a;
    *ke = e < end ? e : end;
}

/* Partial slot of segment (wg, unit s * n_groups + grp). */
LFM_IDX_FN uint64_t lfm_bal_slot(uint32_t wg, uint32_t s, uint32_t n_groups, uint32_t grp) {
    return (uint64_t)wg + (uint64_t)s * n_groups + grp;
}

/* Uniform batch: the unit, group and tile range of workgroup wg < G. */
typedef struct {
    uint32_t s, grp, a, b;
    uint32_t n;    /* workgroups per unit (1: written directly) */
    uint64_t slot;
} lfm_bal_useg;

LFM_IDX_FN lfm_bal_useg lfm_bal_uniform_segment(const lfm_bal_cfg *c, uint32_t wg, uint32_t G, uint32_t tiles) {
    lfm_bal_useg u;
    const uint32_t units = c->n_seq * c->n_groups;
    u.n                  = G / units;
    const uint32_t unit  = wg / u.n, sp = wg - unit * u.n;
    u.s                  = unit / c->n_groups;
    u.grp                = unit - u.s * c->n_groups;
    u.a                  = (uint32_t)((uint64_t)sp * tiles / u.n);
    u.b                  = (uint32_t)((uint64_t)(sp + 1u) * tiles / u.n);
    u.slot               = (uint64_t)wg + unit;
    return u;
}

/* Merge: the workgroups [*g0, *g1] whose partials hold unit (s, grp), for a
 * sequence of `tiles` tiles with `before` tiles (per group) ahead of it;
 * *g0 == *g1 means the unit was written directly.  The partial of workgroup
 * g sits in slot g + s * n_groups + grp. */
LFM_IDX_FN void lfm_bal_merge_range(uint32_t before, uint32_t tiles, uint32_t grp, uint32_t T, uint32_t n_groups,
                                    uint32_t G, uint32_t *g0, uint32_t *g1) {
    const uint64_t N  = (uint64_t)T * n_groups;
    const uint64_t u0 = (uint64_t)before * n_groups + (uint64_t)grp * tiles;
    *g0 = lfm_bal_tile_owner(u0, N, G);
    *g1 = lfm_bal_tile_owner(u0 + tiles - 1u, N, G);
}

/* Partial slots the workspace must hold for a launch of n_wg workgroups. */
LFM_IDX_FN uint64_t lfm_bal_n_slots(uint32_t n_wg, uint32_t n_groups, uint32_t n_seq) {
    return (uint64_t)n_wg + (uint64_t)n_groups * n_seq;
}

/* Workgroups to launch (host): enough for either plan.  keys: an upper bound
 * of the keys a row attends (0 = unknown).  With at most tiles(keys) tiles
 * per sequence a uniform batch needs units * n workgroups, n <=
 * ceil(target_waves / (n_seq * n_head_kv)) and n <= ceil(tiles /
 * min_tiles); a ragged one min(n_res, N / min_tiles).  Without a bound (or
 * with a wrong one) the device plan is capped by the launch, which only makes
 * the shares longer. */
LFM_IDX_FN uint32_t lfm_bal_launch_wgs(const lfm_bal_cfg *c, uint32_t keys) {
    const uint64_t units = (uint64_t)c->n_groups * c->n_seq;
    const uint64_t pairs = (uint64_t)c->n_seq * c->n_head_kv;
    uint64_t per_unit    = (c->target_waves + pairs - 1u) / pairs;
    uint64_t ragged      = c->n_res;
    if (keys) {
        const uint64_t most = (((uint64_t)keys + 31u) / 32u + c->min_tiles - 1u) / c->min_tiles;
        if (per_unit > most) per_unit = most;
        if (ragged > units * most) ragged = units * most;
    }
    uint64_t n = units * per_unit;
    if (n < ragged) n = ragged;
    if (n < units) n = units;
    if (n > 0x1000000u) n = 0x1000000u;
    return (uint32_t)n;
}

#endif /* LFM_SPLITKV_PLAN_H */
