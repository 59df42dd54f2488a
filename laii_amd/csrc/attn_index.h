/*
 * attn_index.h -- integer position / window / ring-slot math of the attention path.
 *
 * One header, compiled into the host launch code and into the HIP kernels
 * (functions are __host__ __device__ under hipcc), so every position, mask
 * bound and ring slot the kernels use is the value the host validated.
 *
 * Semantics follow the reference:
 *   - LFM3 row plan: tools/lfm3_engine.c:862-873 (t_start, count, seg1_slot,
 *     seg1_len, seg2_len; seg2 restarts at slot 0).
 *   - LFM2 rows attend [0, pos] with slot == position
 *     (tools/lfm2_kernels_fast.c:739, tools/lfm2_threadpool.c:787-789).
 *
 * The kernels address keys by absolute position p in [t_start, abs_pos] and
 * map p to a slot with lfm_slot_of(): for a sliding window that is p % cap,
 * which enumerates exactly the slots of seg1 followed by seg2 (seg1 covers
 * slots t_start%cap .. cap-1, seg2 covers 0 .. seg2_len-1).  The CPU tests
 * check this equality exhaustively against the literal segment walk.
 */
#ifndef LFM_ATTN_INDEX_H
#define LFM_ATTN_INDEX_H

#include <stdint.h>

#if defined(__HIPCC__)
#define LFM_IDX_FN __host__ __device__ static inline
#else
#define LFM_IDX_FN static inline
#endif

typedef struct {
    uint32_t t_start;   /* first absolute key position the row attends       */
    uint32_t count;     /* keys attended: abs_pos - t_start + 1 (always >= 1) */
    uint32_t seg1_slot; /* slot of t_start                                    */
    uint32_t seg1_len;  /* keys in the run starting at seg1_slot              */
    uint32_t seg2_len;  /* keys in the wrapped run starting at slot 0         */
} lfm_seg_plan_t;

/* Row plan for a query at absolute position abs_pos.
 * window_len == 0: linear cache, the row attends [0, abs_pos].
 * window_len  > 0: ring of `cap` slots, the row attends the last window_len
 * positions (fewer while abs_pos + 1 < window_len). */
LFM_IDX_FN lfm_seg_plan_t lfm_plan_row(uint32_t abs_pos, uint32_t window_len, uint32_t cap) {
    lfm_seg_plan_t p;
    p.t_start   = (window_len > 0u && abs_pos + 1u > window_len) ? (abs_pos + 1u - window_len) : 0u;
    p.count     = abs_pos - p.t_start + 1u;
    p.seg1_slot = (window_len > 0u) ? (p.t_start % cap) : p.t_start;
    p.seg1_len  = (window_len > 0u && p.seg1_slot + p.count > cap) ? (cap - p.seg1_slot) : p.count;
    p.seg2_len  = p.count - p.seg1_len;
    return p;
}

/* Slot holding absolute position p (valid for p inside the row's window). */
LFM_IDX_FN uint32_t lfm_slot_of(uint32_t p, uint32_t window_len, uint32_t cap) {
    return (window_len > 0u) ? (p % cap) : p;
}

/* Geometry check shared by every entry point: a sliding window must fit in
 * its ring, and every attended slot must lie inside the cache.
 * Returns 0 when rows pos_0 .. pos_0+n_rows-1 are addressable, else -1. */
LFM_IDX_FN int lfm_check_rows(uint32_t pos_0, uint32_t n_rows, uint32_t window_len, uint32_t cap) {
    if (n_rows == 0u) return -1;
    if ((uint64_t)pos_0 + (uint64_t)n_rows - 1u > 0xFFFFFFFEull) return -1;
    if (window_len > 0u) {
        if (cap == 0u || window_len > cap) return -1;
        return 0;
    }
    /* linear cache: cap == 0 means "caller guarantees the cache length" */
    if (cap > 0u && (uint64_t)pos_0 + n_rows > (uint64_t)cap) return -1;
    return 0;
}

#endif /* LFM_ATTN_INDEX_H */
