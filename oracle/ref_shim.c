/*
 * oracle/ref_shim.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Exposes the reference's own CPU attention kernels (compiled from the
 * sources where they lie under /root/reference; nothing is copied) as plain C
 * functions, so tests can pin the oracle restatement against the real thing
 * and bench.py can time the reference as the CPU baseline.  Built by
 * oracle/Makefile into oracle/_ref/libref_attn.so, only where /root/reference
 * exists; the resulting library travels with the tree.
 *
 * The reference pool pins the calling thread and sets FTZ/DAZ on it
 * (tools/lfm2_threadpool.c:384-414); every entry point here restores the
 * caller's affinity mask and MXCSR before returning.
 */
#define _GNU_SOURCE 1
#define LFM2_LOADER_NO_MAIN 1
#define LFM2_THREADPOOL_NO_MAIN 1
#define LFM2_FORWARD_NO_MAIN 1
#define LFM2_DECODE_1X4_NO_MAIN 1
#define LFM2_KERNELS_FAST_NO_MAIN 1
#define LFM2_PREFILL_BATCH_NO_MAIN 1
#define LFM2_SPECULATIVE_PLD_NO_MAIN 1
#define LFM3_ENGINE_NO_MAIN 1
#define LFM2_RUNTIME_FEATURES_NO_MAIN 1
#define LFM2_SYS_CACHE_NO_MAIN 1
#define LFM2_MOE_CHECKPOINT_NO_MAIN 1
#include "tools/lfm3_engine.c"
#include "tools/lfm2_runtime_features.c"
#include "tools/lfm2_sys_cache.c"
#include "tools/lfm2_moe_checkpoint.c"

#include <sched.h>
#include <time.h>
#include <xmmintrin.h>

typedef struct {
    cpu_set_t aff;
    unsigned  csr;
} shim_state;

static void shim_save(shim_state *s) {
    CPU_ZERO(&s->aff);
    sched_getaffinity(0, sizeof s->aff, &s->aff);
    s->csr = _mm_getcsr();
}

static void shim_restore(const shim_state *s) {
    sched_setaffinity(0, sizeof s->aff, &s->aff);
    _mm_setcsr(s->csr);
}

static GGUFTensor shim_f32_tensor(const float *data, uint64_t n) {
    GGUFTensor t;
    memset(&t, 0, sizeof t);
    t.n_dims = 1;
    t.ne[0]  = n;
    t.ne[1] = t.ne[2] = t.ne[3] = 1;
    t.type   = GGML_TYPE_F32;
    t.bytes  = (size_t)n * sizeof(float);
    t.data   = data;
    return t;
}

int ref_has_avx2(void) { return LFM2_HAS_AVX2 ? 1 : 0; }

/* lfm2_rope_lut_init, tools/lfm2_kernels_fast.c:370-388 */
int ref_rope_lut_lfm2(float *cos_out, float *sin_out, uint32_t max_seq, uint32_t head_dim,
                      float freq_base) {
    LFM2RoPELUT lut;
    if (!lfm2_rope_lut_init(&lut, max_seq, head_dim, freq_base)) return -1;
    memcpy(cos_out, lut.cos_lut, (size_t)max_seq * (head_dim / 2) * sizeof(float));
    memcpy(sin_out, lut.sin_lut, (size_t)max_seq * (head_dim / 2) * sizeof(float));
    lfm2_rope_lut_free(&lut);
    return 0;
}

/* lfm3_rope_lut_init, tools/lfm3_engine.c:403-450 */
int ref_rope_lut_lfm3(float *cos_out, float *sin_out, uint32_t max_seq, uint32_t head_dim,
                      uint32_t rope_dim, float freq_base, const float *rope_freqs,
                      uint32_t n_rope_freqs) {
    LFM2RoPELUT lut;
    GGUFTensor rf = shim_f32_tensor(rope_freqs, n_rope_freqs);
    if (!lfm3_rope_lut_init(&lut, max_seq, head_dim, rope_dim, freq_base,
                            rope_freqs ? &rf : NULL)) return -1;
    memcpy(cos_out, lut.cos_lut, (size_t)max_seq * (head_dim / 2) * sizeof(float));
    memcpy(sin_out, lut.sin_lut, (size_t)max_seq * (head_dim / 2) * sizeof(float));
    lfm2_rope_lut_free(&lut);
    return 0;
}

/* Wrap a caller LUT in 64-byte aligned storage (the AVX2 kernels use
 * aligned loads of the cos/sin rows). */
static int shim_lut(LFM2RoPELUT *lut, const float *cos_lut, const float *sin_lut,
                    uint32_t max_seq, uint32_t half) {
    const size_t bytes = (size_t)max_seq * half * sizeof(float);
    lut->max_seq_len = max_seq;
    lut->half_dim    = half;
    lut->cos_lut     = (float *)lfm2_aligned_alloc_64(bytes);
    lut->sin_lut     = (float *)lfm2_aligned_alloc_64(bytes);
    if (!lut->cos_lut || !lut->sin_lut) return -1;
    memcpy(lut->cos_lut, cos_lut, bytes);
    memcpy(lut->sin_lut, sin_lut, bytes);
    return 0;
}

/* lfm2_qk_norm_rope_avx2 (tools/lfm2_kernels_fast.c:403-497) or the scalar
 * kernel (:511-547); head_dim is 64. */
int ref_qk_norm_rope_lfm2(float *vec, uint16_t *dst_f16, uint32_t n_heads, const float *norm_w,
                          float eps, const float *cos_lut, const float *sin_lut,
                          uint32_t max_seq, uint32_t pos, int force_scalar) {
    LFM2RoPELUT lut;
    if (shim_lut(&lut, cos_lut, sin_lut, max_seq, 32u) != 0) return -1;
    GGUFTensor nw = shim_f32_tensor(norm_w, 64u);
#if LFM2_HAS_AVX2
    if (!force_scalar)
        lfm2_qk_norm_rope_avx2(vec, dst_f16, n_heads, 64u, norm_w ? &nw : NULL, eps, &lut, pos);
    else
#endif
        lfm2_qk_norm_rope_scalar(vec, dst_f16, n_heads, 64u, norm_w ? &nw : NULL, eps, &lut, pos);
    lfm2_rope_lut_free(&lut);
    return 0;
}

/* lfm3_qk_norm_rope_simd (tools/lfm3_engine.c:644-666) / scalar (:599-642). */
int ref_qk_norm_rope_lfm3(float *vec, uint16_t *dst_f16, uint32_t n_heads, uint32_t head_dim,
                          const float *norm_w, float eps, const float *cos_lut,
                          const float *sin_lut, uint32_t max_seq, uint32_t pos, int force_scalar) {
    LFM2RoPELUT lut;
    if (shim_lut(&lut, cos_lut, sin_lut, max_seq, head_dim / 2u) != 0) return -1;
    GGUFTensor nw = shim_f32_tensor(norm_w, head_dim);
    if (force_scalar)
        lfm3_qk_norm_rope_scalar(vec, dst_f16, n_heads, head_dim, norm_w ? &nw : NULL, eps, &lut, pos);
    else
        lfm3_qk_norm_rope_simd(vec, dst_f16, n_heads, head_dim, norm_w ? &nw : NULL, eps, &lut, pos);
    lfm2_rope_lut_free(&lut);
    return 0;
}

/* The float-angle RoPE table of the production LFM2 stacks.  which = 0:
 * lfm2_batch_state_init (tools/lfm2_prefill_batch.c:727-736); which = 1:
 * lfm2_state_init (tools/lfm2_forward.c:572-581).  Each state is initialised
 * for a model description carrying only what the table and the state's
 * buffers read (n_embd = n_head_q * head_dim, no layers), the table copied
 * out and the state freed. */
int ref_rope_table_lfm2(float *cos_out, float *sin_out, uint32_t max_seq, uint32_t n_head_q,
                        uint32_t head_dim, float freq_base, int which) {
    LFM2Model *m = (LFM2Model *)calloc(1, sizeof *m);
    if (!m) return -1;
    m->cfg.n_embd         = n_head_q * head_dim;
    m->cfg.n_head_q       = n_head_q;
    m->cfg.head_dim       = head_dim;
    m->cfg.n_vocab        = 256u;
    m->cfg.n_ff           = 256u;
    m->cfg.rope_freq_base = freq_base;
    const size_t bytes    = (size_t)max_seq * (head_dim / 2u) * sizeof(float);
    int rc                = -1;
    shim_state st;
    shim_save(&st);
    if (which == 0) {
        LFM2BatchState *s = (LFM2BatchState *)calloc(1, sizeof *s);
        if (s && lfm2_batch_state_init(s, m, max_seq, 1u) && s->max_seq_len == max_seq) {
            memcpy(cos_out, s->rope_cos, bytes);
            memcpy(sin_out, s->rope_sin, bytes);
            rc = 0;
        }
        if (s) lfm2_batch_state_free(s);
        free(s);
    } else {
        LFM2State *s = (LFM2State *)calloc(1, sizeof *s);
        if (s && lfm2_state_init(s, m, max_seq) && s->max_seq_len == max_seq) {
            memcpy(cos_out, s->rope_cos, bytes);
            memcpy(sin_out, s->rope_sin, bytes);
            rc = 0;
        }
        if (s) lfm2_state_free(s);
        free(s);
    }
    shim_restore(&st);
    free(m);
    return rc;
}

/* The prologue of the production LFM2 stacks on one token, in place:
 * which = 0: lfm2_qk_norm_and_rope_table (tools/lfm2_prefill_batch.c:826-893);
 * which = 1: lfm2_qk_norm_and_rope (tools/lfm2_forward.c:775-830), reading
 * the table through a state that holds only it.  Both run lfm2_rmsnorm
 * (tools/lfm2_forward.c:669-706) per head, then the NeoX rotation. */
int ref_qk_norm_rope_table(float *vec, uint32_t n_heads, uint32_t head_dim, const float *norm_w,
                           float eps, const float *cos_tab, const float *sin_tab, uint32_t pos,
                           int which) {
    GGUFTensor nw = shim_f32_tensor(norm_w, head_dim);
    if (which == 0) {
        lfm2_qk_norm_and_rope_table(cos_tab, sin_tab, vec, n_heads, head_dim, norm_w ? &nw : NULL, eps, pos);
    } else {
        LFM2State *s = (LFM2State *)calloc(1, sizeof *s);
        if (!s) return -1;
        s->rope_cos = (float *)cos_tab;
        s->rope_sin = (float *)sin_tab;
        lfm2_qk_norm_and_rope(s, vec, n_heads, head_dim, norm_w ? &nw : NULL, eps, pos);
        free(s);
    }
    return 0;
}

/* lfm2_store_fp32_to_fp16_simd (tools/lfm2_kernels_fast.c:500-507) */
void ref_store_fp32_to_fp16(uint16_t *dst, const float *src, uint32_t n) {
    uint32_t i = 0;
#if LFM2_HAS_AVX2
    for (; i + 8u <= n; i += 8u) lfm2_store_fp32_to_fp16_avx2(dst + i, src + i, 8u);
#endif
    for (; i < n; ++i) dst[i] = fp32_to_fp16(src[i]);
}

float ref_fp16_to_fp32(uint16_t h) { return lfm2_fp16_to_fp32(h); }

/* OnlineGQATaskCtx + lfm2_parallel_for (tools/lfm2_kernels_fast.c:1052-1066). */
void ref_online_gqa_f16(const float *q, const uint16_t *k16, const uint16_t *v16, float *out,
                        uint32_t n_head_q, uint32_t kv_mul, uint32_t kv_dim, uint32_t pos,
                        uint32_t n_threads) {
    shim_state st;
    shim_save(&st);
    LFM2ThreadPool pool;
    lfm2_threadpool_init(&pool, n_threads);
    OnlineGQATaskCtx ctx = {
        .pool = &pool, .q = q, .k_cache_f16 = k16, .v_cache_f16 = v16, .xb_out = out,
        .xb_q8_out = NULL, .n_head_q = n_head_q, .kv_mul = kv_mul, .kv_dim = kv_dim,
        .pos = pos, .scale = 1.0f / sqrtf(64.0f)};
    lfm2_parallel_for(&pool, (n_head_q + 3u) / 4u, 1, lfm2_online_gqa_f16_worker_simd, &ctx);
    lfm2_threadpool_free(&pool);
    shim_restore(&st);
}

/* GQAAttnTaskCtx + lfm2_gqa_heads_worker_task (tools/lfm2_prefill_batch.c:1074-1091);
 * f16 caches NULL selects the FP32 two-pass branch. */
void ref_gqa_heads(const float *q, const float *k32, const float *v32, const uint16_t *k16,
                   const uint16_t *v16, float *out, uint32_t n_head_q, uint32_t kv_mul,
                   uint32_t head_dim, uint32_t kv_dim, uint32_t max_seq, uint32_t pos,
                   uint32_t n_threads) {
    shim_state st;
    shim_save(&st);
    LFM2ThreadPool pool;
    lfm2_threadpool_init(&pool, n_threads);
    float *att = (float *)calloc((size_t)n_head_q * max_seq, sizeof(float));
    GQAAttnTaskCtx ctx = {
        .pool = &pool, .q = q, .k_cache = k32, .v_cache = v32, .k_cache_f16 = k16,
        .v_cache_f16 = v16, .att = att, .xb = out, .n_head_q = n_head_q, .kv_mul = kv_mul,
        .head_dim = head_dim, .kv_dim = kv_dim, .max_seq_len = max_seq, .pos = pos,
        .scale = 1.0f / sqrtf((float)head_dim)};
    lfm2_parallel_for(&pool, n_head_q, 1, lfm2_gqa_heads_worker_task, &ctx);
    free(att);
    lfm2_threadpool_free(&pool);
    shim_restore(&st);
}

/* lfm3_online_gqa_f16_dispatch (tools/lfm3_engine.c:1155-1204). */
void ref_lfm3_dispatch(const float *q, const float *gate, const uint16_t *k16, const uint16_t *v16,
                       float *out, uint32_t B, uint32_t pos_0, uint32_t window_len,
                       uint32_t swa_cap, uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                       uint32_t n_threads) {
    shim_state st;
    shim_save(&st);
    LFM2ThreadPool pool;
    lfm2_threadpool_init(&pool, n_threads);
    lfm3_online_gqa_f16_dispatch(&pool, q, gate, k16, v16, out, NULL, B, pos_0, window_len,
                                 swa_cap, n_head_q, n_head_kv, head_dim);
    lfm2_threadpool_free(&pool);
    shim_restore(&st);
}

static double shim_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* CPU baseline, reference-faithful: one pool, each sequence dispatched as
 * the engine dispatches one decode step (ceil(n_head_q/4) items,
 * tools/lfm2_kernels_fast.c:1065-1066), sequences one after another.
 * head_dim is 64.  Runs `reps` passes and returns the seconds of the fastest;
 * *threads_out receives the pool's actual worker count. */
double ref_time_decode_batch(const float *q, const uint16_t *const *k_seq,
                             const uint16_t *const *v_seq, const uint32_t *pos, float *out,
                             uint32_t n_seq, uint32_t n_head_q, uint32_t n_head_kv,
                             uint32_t n_threads, uint32_t reps, uint32_t *threads_out) {
    shim_state st;
    shim_save(&st);
    LFM2ThreadPool pool;
    lfm2_threadpool_init(&pool, n_threads);
    if (threads_out) *threads_out = pool.n_threads;
    const uint32_t kv_dim = n_head_kv * 64u;
    double best = 1e30;
    for (uint32_t r = 0; r < reps; ++r) {
        const double t0 = shim_now();
        for (uint32_t s = 0; s < n_seq; ++s) {
            OnlineGQATaskCtx ctx = {
                .pool = &pool, .q = q + (size_t)s * n_head_q * 64u, .k_cache_f16 = k_seq[s],
                .v_cache_f16 = v_seq[s], .xb_out = out + (size_t)s * n_head_q * 64u,
                .xb_q8_out = NULL, .n_head_q = n_head_q, .kv_mul = n_head_q / n_head_kv,
                .kv_dim = kv_dim, .pos = pos[s], .scale = 1.0f / sqrtf(64.0f)};
            lfm2_parallel_for(&pool, (n_head_q + 3u) / 4u, 1, lfm2_online_gqa_f16_worker_simd,
                              &ctx);
        }
        const double dt = shim_now() - t0;
        if (dt < best) best = dt;
    }
    lfm2_threadpool_free(&pool);
    shim_restore(&st);
    return best;
}

/* CPU baseline, fair-batched: the reference's decode worker on every
 * (sequence, 4-head group) item of the batch, claimed dynamically by
 * n_threads threads (FTZ/DAZ set as the reference pool sets them,
 * tools/lfm2_threadpool.c:384-414), so all cores stay busy across sequences.
 * Each item hands the worker a one-item claim range (the fields that
 * lfm2_threadpool_claim_chunk reads, tools/lfm2_threadpool.c:506-520), so the
 * worker computes exactly that group.  head_dim is 64. */
typedef struct {
    const float *q;
    const uint16_t *const *k_seq;
    const uint16_t *const *v_seq;
    const uint32_t *pos;
    float *out;
    uint32_t n_seq, n_head_q, n_head_kv, n_groups;
    atomic_uint next;
} fair_job;

static void *fair_worker(void *arg) {
    fair_job *j = (fair_job *)arg;
    _mm_setcsr(_mm_getcsr() | 0x8040u);
    LFM2ThreadPool one;
    memset(&one, 0, sizeof one);
    one.chunk_size = 1u;
    for (;;) {
        const uint32_t it = atomic_fetch_add_explicit(&j->next, 1u, memory_order_relaxed);
        if (it >= j->n_seq * j->n_groups) break;
        const uint32_t s = it / j->n_groups, g = it % j->n_groups;
        one.n_items = g + 1u;
        atomic_store_explicit(&one.next_item, g, memory_order_relaxed);
        OnlineGQATaskCtx ctx = {
            .pool = &one, .q = j->q + (size_t)s * j->n_head_q * 64u, .k_cache_f16 = j->k_seq[s],
            .v_cache_f16 = j->v_seq[s], .xb_out = j->out + (size_t)s * j->n_head_q * 64u,
            .xb_q8_out = NULL, .n_head_q = j->n_head_q, .kv_mul = j->n_head_q / j->n_head_kv,
            .kv_dim = j->n_head_kv * 64u, .pos = j->pos[s], .scale = 1.0f / sqrtf(64.0f)};
        lfm2_online_gqa_f16_worker_simd(&ctx, 0u, 1u);
    }
    return NULL;
}

double ref_time_decode_batch_fair(const float *q, const uint16_t *const *k_seq,
                                  const uint16_t *const *v_seq, const uint32_t *pos, float *out,
                                  uint32_t n_seq, uint32_t n_head_q, uint32_t n_head_kv,
                                  uint32_t n_threads, uint32_t reps) {
    shim_state st;
    shim_save(&st);
    if (n_threads < 1u) n_threads = 1u;
    if (n_threads > 256u) n_threads = 256u;
    double best = 1e30;
    for (uint32_t r = 0; r < reps; ++r) {
        fair_job job = {q, k_seq, v_seq, pos, out, n_seq, n_head_q, n_head_kv, (n_head_q + 3u) / 4u, 0u};
        pthread_t th[256];
        const double t0 = shim_now();
        for (uint32_t t = 1; t < n_threads; ++t) pthread_create(&th[t], NULL, fair_worker, &job);
        fair_worker(&job);
        for (uint32_t t = 1; t < n_threads; ++t) pthread_join(th[t], NULL);
        const double dt = shim_now() - t0;
        if (dt < best) best = dt;
    }
    shim_restore(&st);
    return best;
}

/* ---- CPU baseline of every decode-type configuration --------------------
 * kind 0  LFM2 decode, one query row per sequence: OnlineGQATaskCtx +
 *         lfm2_online_gqa_f16_worker_simd over ceil(n_head_q / 4) head groups
 *         (tools/lfm2_kernels_fast.c:1052-1066); head_dim 64.
 * kind 1  LFM2 causal rows (speculative verify, prefill): per row,
 *         GQAAttnTaskCtx + lfm2_gqa_heads_worker_task over the query heads
 *         (tools/lfm2_prefill_batch.c:1074-1091); row r of sequence s at
 *         pos0[s] + r; head_dim 64.
 * kind 2  LFM3 decode, one row per sequence: lfm3_online_gqa_f16_dispatch
 *         with B = 1 (tools/lfm3_engine.c:1155-1204), B * n_head_q / 2 items;
 *         gate (sigmoid values, [n_seq][n_head_q]) or NULL.
 * fair 0  reference-faithful: the engine's dispatch on one pool of n_threads
 *         (the calling thread is worker 0), sequence after sequence (row
 *         after row for kind 1), as a multi-sequence batch would run on it;
 * fair 1  fair-batched: every (sequence, row, item) of the batch claimed
 *         dynamically by n_threads threads (FTZ/DAZ as the pool sets them),
 *         each handing the reference worker a one-item claim range.
 * Runs `warm` untimed passes, then `reps` timed ones; times_out[r] receives
 * pass r's seconds, *threads_out the threads used. */
typedef struct {
    int kind;
    const float *q, *gate;
    const uint16_t *const *k_seq;
    const uint16_t *const *v_seq;
    const uint32_t *pos0;
    float *out;
    uint32_t n_seq, n_rows, n_head_q, n_head_kv, head_dim, window, cap, max_seq;
    uint32_t per_seq; /* items per sequence */
    atomic_uint next;
    /* fair mode: persistent threads, one start and one end barrier per pass */
    pthread_barrier_t start, end;
    uint32_t passes;
} attn_job;

static uint32_t attn_items_per_seq(const attn_job *j) {
    if (j->kind == 0) return (j->n_head_q + 3u) / 4u;
    if (j->kind == 1) return j->n_rows * j->n_head_q;
    return j->head_dim == 128u ? (j->n_head_q + 1u) / 2u : j->n_head_q;
}

/* one == 0: the engine's dispatch of sequence s (of row `item` for kind 1)
 * on the real pool `pool`; one != 0: item `item` of sequence s alone, through
 * the one-item claim range `pool`.  att: the heads task's score scratch. */
static void attn_run(const attn_job *j, LFM2ThreadPool *pool, uint32_t s, uint32_t item, int one, float *att) {
    const uint32_t hd = j->head_dim, kv_dim = j->n_head_kv * hd;
    if (j->kind == 0) {
        OnlineGQATaskCtx ctx = {
            .pool = pool, .q = j->q + (size_t)s * j->n_head_q * hd, .k_cache_f16 = j->k_seq[s],
            .v_cache_f16 = j->v_seq[s], .xb_out = j->out + (size_t)s * j->n_head_q * hd, .xb_q8_out = NULL,
            .n_head_q = j->n_head_q, .kv_mul = j->n_head_q / j->n_head_kv, .kv_dim = kv_dim, .pos = j->pos0[s],
            .scale = 1.0f / sqrtf((float)hd)};
        if (one) lfm2_online_gqa_f16_worker_simd(&ctx, 0u, 1u);
        else lfm2_parallel_for(pool, (j->n_head_q + 3u) / 4u, 1, lfm2_online_gqa_f16_worker_simd, &ctx);
    } else if (j->kind == 1) {
        const uint32_t r  = one ? item / j->n_head_q : item;
        const size_t row  = ((size_t)s * j->n_rows + r) * j->n_head_q * hd;
        GQAAttnTaskCtx ctx = {
            .pool = pool, .q = j->q + row, .k_cache = NULL, .v_cache = NULL, .k_cache_f16 = j->k_seq[s],
            .v_cache_f16 = j->v_seq[s], .att = att, .xb = j->out + row, .n_head_q = j->n_head_q,
            .kv_mul = j->n_head_q / j->n_head_kv, .head_dim = hd, .kv_dim = kv_dim, .max_seq_len = j->max_seq,
            .pos = j->pos0[s] + r, .scale = 1.0f / sqrtf((float)hd)};
        if (one) lfm2_gqa_heads_worker_task(&ctx, 0u, 1u);
        else lfm2_parallel_for(pool, j->n_head_q, 1, lfm2_gqa_heads_worker_task, &ctx);
    } else {
        const float *g = j->gate ? j->gate + (size_t)s * j->n_head_q : NULL;
        if (!one) {
            lfm3_online_gqa_f16_dispatch(pool, j->q + (size_t)s * j->n_head_q * hd, g, j->k_seq[s], j->v_seq[s],
                                         j->out + (size_t)s * j->n_head_q * hd, NULL, 1u, j->pos0[s], j->window,
                                         j->cap, j->n_head_q, j->n_head_kv, hd);
            return;
        }
        const uint32_t per = hd == 128u ? 2u : 1u;
        LFM3OnlineGQACtx ctx = {
            .pool = pool, .q_batch = j->q + (size_t)s * j->n_head_q * hd, .gate_sig = g,
            .k_cache_f16 = j->k_seq[s], .v_cache_f16 = j->v_seq[s], .xb_out = j->out + (size_t)s * j->n_head_q * hd,
            .xb_q8_out = NULL, .B = 1u, .pos_0 = j->pos0[s], .window_len = j->window, .swa_cap = j->cap,
            .n_head_q = j->n_head_q, .kv_mul = j->n_head_q / j->n_head_kv, .kv_dim = kv_dim, .head_dim = hd,
            .n_groups = (j->n_head_q + per - 1u) / per, .scale = 1.0f / sqrtf((float)hd)};
#if LFM2_HAS_AVX2
        if (hd == 128u && lfm3_use_avx2()) {
            lfm3_online_gqa_128_f16_worker_avx2(&ctx, 0u, 1u);
            return;
        }
#endif
        lfm3_online_gqa_f16_worker_scalar(&ctx, 0u, 1u);
    }
}

/* One fair pass: items claimed until the batch is done. */
static void attn_fair_pass(attn_job *j, float *att) {
    LFM2ThreadPool one;
    memset(&one, 0, sizeof one);
    one.chunk_size = 1u;
    for (;;) {
        const uint32_t it = atomic_fetch_add_explicit(&j->next, 1u, memory_order_relaxed);
        if (it >= j->n_seq * j->per_seq) break;
        const uint32_t s = it / j->per_seq, item = it % j->per_seq;
        /* the worker claims exactly `sub` from a range that ends after it */
        const uint32_t sub = j->kind == 1 ? item % j->n_head_q : item;
        one.n_items = sub + 1u;
        atomic_store_explicit(&one.next_item, sub, memory_order_relaxed);
        attn_run(j, &one, s, item, 1, att);
    }
}

/* A helper thread of the fair mode: every pass between the two barriers. */
static void *attn_fair_thread(void *arg) {
    attn_job *j = (attn_job *)arg;
    _mm_setcsr(_mm_getcsr() | 0x8040u);
    float *att = (float *)calloc((size_t)j->n_head_q * (j->max_seq ? j->max_seq : 1u), sizeof(float));
    for (uint32_t r = 0; r < j->passes; ++r) {
        pthread_barrier_wait(&j->start);
        attn_fair_pass(j, att);
        pthread_barrier_wait(&j->end);
    }
    free(att);
    return NULL;
}

int ref_time_attn(int kind, int fair, const float *q, const float *gate, const uint16_t *const *k_seq,
                  const uint16_t *const *v_seq, const uint32_t *pos0, float *out, uint32_t n_seq, uint32_t n_rows,
                  uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim, uint32_t window, uint32_t cap,
                  uint32_t max_seq, uint32_t n_threads, uint32_t warm, uint32_t reps, double *times_out,
                  uint32_t *threads_out) {
    if (kind < 0 || kind > 2 || n_seq == 0u || n_head_kv == 0u || n_head_q % n_head_kv != 0u) return -1;
    if (kind != 2 && head_dim != 64u) return -1;
    if (n_threads < 1u) n_threads = 1u;
    if (n_threads > 256u) n_threads = 256u;
    static attn_job job; /* one timing at a time (the barriers live in it) */
    memset(&job, 0, sizeof job);
    job.kind = kind, job.q = q, job.gate = gate, job.k_seq = k_seq, job.v_seq = v_seq, job.pos0 = pos0;
    job.out = out, job.n_seq = n_seq, job.n_rows = kind == 1 ? n_rows : 1u, job.n_head_q = n_head_q;
    job.n_head_kv = n_head_kv, job.head_dim = head_dim, job.window = window, job.cap = cap;
    job.max_seq = max_seq, job.passes = warm + reps;
    job.per_seq = attn_items_per_seq(&job);
    shim_state st;
    shim_save(&st);
    LFM2ThreadPool pool;
    pthread_t th[256];
    float *att = (float *)calloc((size_t)n_head_q * (max_seq ? max_seq : 1u), sizeof(float));
    if (!fair) {
        lfm2_threadpool_init(&pool, n_threads);
        if (threads_out) *threads_out = pool.n_threads;
    } else {
        if (threads_out) *threads_out = n_threads;
        _mm_setcsr(_mm_getcsr() | 0x8040u);
        pthread_barrier_init(&job.start, NULL, n_threads);
        pthread_barrier_init(&job.end, NULL, n_threads);
        for (uint32_t t = 1; t < n_threads; ++t) pthread_create(&th[t], NULL, attn_fair_thread, &job);
    }
    for (uint32_t r = 0; r < warm + reps; ++r) {
        atomic_store(&job.next, 0u);
        const double t0 = shim_now();
        if (!fair) {
            for (uint32_t s = 0; s < n_seq; ++s)
                for (uint32_t row = 0; row < job.n_rows; ++row) attn_run(&job, &pool, s, row, 0, att);
        } else {
            pthread_barrier_wait(&job.start);
            attn_fair_pass(&job, att);
            pthread_barrier_wait(&job.end);
        }
        const double dt = shim_now() - t0;
        if (r >= warm) times_out[r - warm] = dt;
    }
    if (!fair) {
        lfm2_threadpool_free(&pool);
    } else {
        for (uint32_t t = 1; t < n_threads; ++t) pthread_join(th[t], NULL);
        pthread_barrier_destroy(&job.start);
        pthread_barrier_destroy(&job.end);
    }
    free(att);
    shim_restore(&st);
    return 0;
}

/* ---- attention-sink eviction ------------------------------------------ */
/* A model description carrying only what the shift functions read:
 * n_layers, head_dim (n_embd / n_head_q for LFM2), n_head_kv, sliding_window
 * and each layer's block type. */
static LFM2Model *shim_model(uint32_t n_layers, const uint32_t *n_head_kv,
                             const uint8_t *layer_kind, uint32_t head_dim,
                             uint32_t sliding_window) {
    if (n_layers > LFM2_MAX_LAYERS) return NULL;
    LFM2Model *m = (LFM2Model *)calloc(1, sizeof *m);
    if (!m) return NULL;
    m->cfg.n_layers       = n_layers;
    m->cfg.n_head_q       = 1;
    m->cfg.n_embd         = head_dim;
    m->cfg.head_dim       = head_dim;
    m->cfg.sliding_window = sliding_window;
    for (uint32_t l = 0; l < n_layers; ++l) {
        m->cfg.n_head_kv[l] = n_head_kv[l];
        const uint8_t kind  = layer_kind ? layer_kind[l] : (n_head_kv[l] ? 1u : 0u);
        m->layers[l].block_type = kind == 0u ? LFM2_BLOCK_SHORTCONV
                                : kind == 2u ? LFM2_BLOCK_SWA_ATTN : LFM2_BLOCK_GQA_ATTN;
    }
    return m;
}

/* lfm2_kv_cache_shift_sinks_avx2, tools/lfm2_runtime_features.c:744-833 */
uint32_t ref_kv_shift_sinks_lfm2(uint16_t **k_caches, uint16_t **v_caches, uint32_t n_layers,
                                 const uint32_t *n_head_kv, uint32_t head_dim, float *cos_lut,
                                 float *sin_lut, uint32_t lut_rows, uint32_t pos, uint32_t n_sink,
                                 uint32_t n_discard) {
    LFM2Model *m = shim_model(n_layers, n_head_kv, NULL, head_dim, 0);
    if (!m) return 0xFFFFFFFFu;
    uint16_t *kc[LFM2_MAX_LAYERS] = {0}, *vc[LFM2_MAX_LAYERS] = {0};
    for (uint32_t l = 0; l < n_layers; ++l) { kc[l] = k_caches[l]; vc[l] = v_caches[l]; }
    LFM2RoPELUT lut = {lut_rows, head_dim / 2u, cos_lut, sin_lut};
    shim_state st;
    shim_save(&st);
    lfm2_kv_cache_shift_sinks_avx2(kc, vc, m, &lut, &pos, n_sink, n_discard);
    shim_restore(&st);
    free(m);
    return pos;
}

/* lfm3_kv_cache_shift_sinks, tools/lfm2_runtime_features.c:1055-1163 */
uint32_t ref_kv_shift_sinks_lfm3(uint16_t **k_caches, uint16_t **v_caches, uint32_t n_layers,
                                 const uint32_t *n_head_kv, const uint8_t *layer_kind,
                                 uint32_t head_dim, float *cos_full, float *sin_full,
                                 uint32_t full_rows, float *cos_swa, float *sin_swa,
                                 uint32_t swa_rows, uint32_t sliding_window, uint32_t swa_cap,
                                 uint32_t pos, uint32_t n_sink, uint32_t n_discard) {
    LFM2Model *m = shim_model(n_layers, n_head_kv, layer_kind, head_dim, sliding_window);
    if (!m) return 0xFFFFFFFFu;
    uint16_t *kc[LFM2_MAX_LAYERS] = {0}, *vc[LFM2_MAX_LAYERS] = {0};
    for (uint32_t l = 0; l < n_layers; ++l) { kc[l] = k_caches[l]; vc[l] = v_caches[l]; }
    LFM2RoPELUT lf = {full_rows, head_dim / 2u, cos_full, sin_full};
    LFM2RoPELUT ls = {swa_rows, head_dim / 2u, cos_swa, sin_swa};
    shim_state st;
    shim_save(&st);
    lfm3_kv_cache_shift_sinks(kc, vc, m, &lf, &ls, swa_cap, &pos, n_sink, n_discard);
    shim_restore(&st);
    free(m);
    return pos;
}

/* ---- next-row projections -------------------------------------------------- */

static GGUFTensor shim_q4K_tensor(const void *w, uint32_t n_rows, uint32_t n_cols) {
    GGUFTensor t;
    memset(&t, 0, sizeof t);
    t.n_dims = 2;
    t.ne[0]  = n_cols;
    t.ne[1]  = n_rows;
    t.ne[2] = t.ne[3] = 1;
    t.type   = GGML_TYPE_Q4_K;
    t.bytes  = (size_t)n_rows * (n_cols / 256u) * sizeof(block_q4_K_t);
    t.data   = w;
    return t;
}

/* lfm2_quantize_batch_q8_K_avx2 (tools/lfm2_prefill_batch.c:93-105): the
 * engine's kernel table quantizer (lfm2_quantize_row_q8_K_avx2_cpuid). */
void ref_quantize_q8_K(const float *x, void *y, uint32_t n_rows, uint32_t n_cols) {
    shim_state st;
    shim_save(&st);
    lfm2_quantize_batch_q8_K_avx2(x, (block_q8_K_t *)y, n_rows, n_cols);
    shim_restore(&st);
}

/* lfm2_vec_dot_q4_K_q8_K_avx2 (include/lfm2_simd_avx2.h:364-412), one row. */
float ref_dot_q4_K_avx2(const void *w_row, const void *x_q8, uint32_t n_cols) {
    return lfm2_vec_dot_q4_K_q8_K_avx2((const block_q4_K_t *)w_row, (const block_q8_K_t *)x_q8, n_cols);
}

/* lfm2_matmul_1x4_prequant_mt (tools/lfm2_decode_1x4.c:795-813) without a
 * pool: the engine's decode-step projection from a prequantized vector. */
void ref_matmul_q4_K_prequant(float *out, const void *w, uint32_t n_rows, uint32_t n_cols,
                              const void *x_q8) {
    GGUFTensor t = shim_q4K_tensor(w, n_rows, n_cols);
    shim_state st;
    shim_save(&st);
    lfm2_matmul_1x4_prequant_mt(NULL, out, &t, NULL, (const block_q8_K_t *)x_q8);
    shim_restore(&st);
}

/* lfm2_matmul_batch_avx2_mt (tools/lfm2_prefill_batch.c:598-634) without a
 * pool: quantizes the B <= 8 fp32 tokens, then one row at a time. */
void ref_matmul_q4_K_batch(float *out, const void *w, uint32_t n_rows, uint32_t n_cols,
                           const float *x, uint32_t n_tokens) {
    GGUFTensor t = shim_q4K_tensor(w, n_rows, n_cols);
    block_q8_K_t *scratch = (block_q8_K_t *)malloc((size_t)n_tokens * (n_cols / 256u) * sizeof(block_q8_K_t));
    if (!scratch) return;
    shim_state st;
    shim_save(&st);
    lfm2_matmul_batch_avx2_mt(NULL, out, &t, x, n_tokens, scratch);
    shim_restore(&st);
    free(scratch);
}

/* lfm2_vec_dot_q6_K_q8_K_avx2 (include/lfm2_simd_avx2.h:551-634), one row. */
float ref_dot_q6_K_avx2(const void *w_row, const void *x_q8, uint32_t n_cols) {
    return lfm2_vec_dot_q6_K_q8_K_avx2((const block_q6_K_t *)w_row, (const block_q8_K_t *)x_q8, n_cols);
}

/* ---- prompt cache (.lfmcache v1) ------------------------------------------------ */

static LFM2Model *shim_cache_model(uint32_t n_layers, const uint32_t *n_head_kv, const uint8_t *layer_kind,
                                   uint32_t head_dim, uint32_t n_embd, uint32_t n_head_q,
                                   uint32_t l_cache, uint32_t sliding_window, int is_lfm3) {
    LFM2Model *m = shim_model(n_layers, n_head_kv, layer_kind, head_dim, sliding_window);
    if (!m) return NULL;
    snprintf(m->cfg.arch, sizeof m->cfg.arch, "%s", is_lfm3 ? "lfm3" : "lfm2");
    m->cfg.is_lfm3           = is_lfm3 != 0;
    m->cfg.n_embd            = n_embd;
    m->cfg.n_head_q          = n_head_q;
    m->cfg.shortconv_l_cache = l_cache;
    m->cfg.n_vocab           = 65536;
    for (uint32_t l = 0; l < n_layers; ++l) m->cfg.is_swa_layer[l] = layer_kind && layer_kind[l] == 2u;
    return m;
}

/* lfm2_compute_model_fingerprint (tools/lfm2_sys_cache.c:394-422) of that model */
uint64_t ref_model_fingerprint(uint32_t n_layers, const uint32_t *n_head_kv, const uint8_t *layer_kind,
                               uint32_t head_dim, uint32_t n_embd, uint32_t n_head_q, uint32_t l_cache,
                               uint32_t sliding_window, int is_lfm3) {
    LFM2Model *m = shim_cache_model(n_layers, n_head_kv, layer_kind, head_dim, n_embd, n_head_q, l_cache,
                                    sliding_window, is_lfm3);
    if (!m) return 0;
    const uint64_t h = lfm2_compute_model_fingerprint(m);
    free(m);
    return h;
}

/* lfm2_prompt_cache_save_ex (tools/lfm2_sys_cache.c:504-627) */
int ref_prompt_cache_save(const char *path, uint32_t n_layers, const uint32_t *n_head_kv,
                          const uint8_t *layer_kind, uint32_t head_dim, uint32_t n_embd, uint32_t n_head_q,
                          uint32_t l_cache, uint32_t sliding_window, int is_lfm3, const uint32_t *tokens,
                          uint32_t n_tokens, float **conv, const uint32_t *conv_heads, uint16_t **k,
                          uint16_t **v, uint32_t swa_cap) {
    LFM2Model *m = shim_cache_model(n_layers, n_head_kv, layer_kind, head_dim, n_embd, n_head_q, l_cache,
                                    sliding_window, is_lfm3);
    if (!m) return 0;
    float *cs[LFM2_MAX_LAYERS]    = {0};
    uint16_t *kc[LFM2_MAX_LAYERS] = {0}, *vc[LFM2_MAX_LAYERS] = {0};
    for (uint32_t l = 0; l < n_layers; ++l) { cs[l] = conv[l]; kc[l] = k[l]; vc[l] = v[l]; }
    const bool ok = lfm2_prompt_cache_save_ex(path, m, tokens, n_tokens, cs, conv_heads, kc, vc, swa_cap);
    free(m);
    return ok ? 1 : 0;
}

/* lfm2_prompt_cache_try_load_prefix_ex (tools/lfm2_sys_cache.c:650-797); returns the matched
 * position (0: not applied) */
uint32_t ref_prompt_cache_load(const char *path, uint32_t n_layers, const uint32_t *n_head_kv,
                               const uint8_t *layer_kind, uint32_t head_dim, uint32_t n_embd,
                               uint32_t n_head_q, uint32_t l_cache, uint32_t sliding_window, int is_lfm3,
                               const uint32_t *prompt, uint32_t n_prompt, uint32_t max_seq, float **conv,
                               uint32_t *conv_heads, uint16_t **k, uint16_t **v, uint32_t swa_cap) {
    LFM2Model *m = shim_cache_model(n_layers, n_head_kv, layer_kind, head_dim, n_embd, n_head_q, l_cache,
                                    sliding_window, is_lfm3);
    if (!m) return 0;
    float *cs[LFM2_MAX_LAYERS]    = {0};
    uint16_t *kc[LFM2_MAX_LAYERS] = {0}, *vc[LFM2_MAX_LAYERS] = {0};
    for (uint32_t l = 0; l < n_layers; ++l) { cs[l] = conv[l]; kc[l] = k[l]; vc[l] = v[l]; }
    uint32_t pos = 0;
    (void)lfm2_prompt_cache_try_load_prefix_ex(path, m, prompt, n_prompt, max_seq, cs, conv_heads, kc, vc,
                                               swa_cap, &pos);
    free(m);
    return pos;
}

/* ---- checkpoint SWA slab ------------------------------------------------------ */

/* lfm2_checkpoint_init + lfm2_checkpoint_save_ex (tools/lfm2_moe_checkpoint.c:399-505)
 * of the caches; the slab (swa_total_u16 elements, returned) is copied to slab_out
 * when it is non-NULL. */
size_t ref_checkpoint_swa_save(uint16_t *slab_out, uint32_t n_layers, const uint32_t *n_head_kv,
                               const uint8_t *layer_kind, uint32_t head_dim, uint32_t n_embd,
                               uint32_t n_head_q, uint32_t l_cache, uint32_t sliding_window,
                               uint16_t **k, uint16_t **v) {
    LFM2Model *m = shim_cache_model(n_layers, n_head_kv, layer_kind, head_dim, n_embd, n_head_q, l_cache,
                                    sliding_window, 1);
    if (!m) return 0;
    LFM2Checkpoint cp;
    size_t n = 0;
    if (lfm2_checkpoint_init(&cp, m, 0U)) {
        uint16_t *kc[LFM2_MAX_LAYERS] = {0}, *vc[LFM2_MAX_LAYERS] = {0};
        for (uint32_t l = 0; l < n_layers; ++l) { kc[l] = k[l]; vc[l] = v[l]; }
        lfm2_checkpoint_save_ex(&cp, m, NULL, NULL, kc, vc, 0U, 0ULL, NULL, 0U);
        n = cp.swa_total_u16;
        if (slab_out && n) memcpy(slab_out, cp.swa_kv_slab, n * sizeof(uint16_t));
        lfm2_checkpoint_destroy(&cp);
    }
    free(m);
    return n;
}

/* lfm2_checkpoint_restore_ex (tools/lfm2_moe_checkpoint.c:508-560) from a slab. */
int ref_checkpoint_swa_restore(const uint16_t *slab, uint32_t n_layers, const uint32_t *n_head_kv,
                               const uint8_t *layer_kind, uint32_t head_dim, uint32_t n_embd,
                               uint32_t n_head_q, uint32_t l_cache, uint32_t sliding_window,
                               uint16_t **k, uint16_t **v) {
    LFM2Model *m = shim_cache_model(n_layers, n_head_kv, layer_kind, head_dim, n_embd, n_head_q, l_cache,
                                    sliding_window, 1);
    if (!m) return 0;
    LFM2Checkpoint cp;
    int ok = 0;
    if (lfm2_checkpoint_init(&cp, m, 0U)) {
        if (cp.swa_total_u16) memcpy(cp.swa_kv_slab, slab, cp.swa_total_u16 * sizeof(uint16_t));
        cp.is_valid                   = true;
        uint16_t *kc[LFM2_MAX_LAYERS] = {0}, *vc[LFM2_MAX_LAYERS] = {0};
        for (uint32_t l = 0; l < n_layers; ++l) { kc[l] = k[l]; vc[l] = v[l]; }
        uint32_t pos = 0;
        ok = lfm2_checkpoint_restore_ex(&cp, m, NULL, NULL, kc, vc, &pos, NULL, NULL, NULL) ? 1 : 0;
        lfm2_checkpoint_destroy(&cp);
    }
    free(m);
    return ok;
}

/* ---- other weight types of the decode projection (AVX2 1x1 kernels) ----------- */
/* lfm2_vec_dot_q4_0_q8_K_avx2 (tools/lfm2_cpuid_quants.c:634-672) */
float ref_dot_q4_0_avx2(const void *w_row, const void *x_q8, uint32_t n_cols) {
    return lfm2_vec_dot_q4_0_q8_K_avx2(w_row, (const block_q8_K_t *)x_q8, n_cols);
}
/* lfm2_vec_dot_q8_0_q8_K_avx2 (include/lfm2_simd_avx2.h:639-674) */
float ref_dot_q8_0_avx2(const void *w_row, const void *x_q8, uint32_t n_cols) {
    return lfm2_vec_dot_q8_0_q8_K_avx2((const block_q8_0_t *)w_row, (const block_q8_K_t *)x_q8, n_cols);
}
/* lfm2_vec_dot_q5_K_q8_K_avx2 (tools/lfm2_cpuid_quants.c:690-740) */
float ref_dot_q5_K_avx2(const void *w_row, const void *x_q8, uint32_t n_cols) {
    return lfm2_vec_dot_q5_K_q8_K_avx2(w_row, (const block_q8_K_t *)x_q8, n_cols);
}
/* lfm2_vec_dot_iq4_xs_q8_K_avx2 (tools/lfm2_cpuid_quants.c:832-880) */
float ref_dot_iq4_xs_avx2(const void *w_row, const void *x_q8, uint32_t n_cols) {
    return lfm2_vec_dot_iq4_xs_q8_K_avx2(w_row, (const block_q8_K_t *)x_q8, n_cols);
}
/* the engine's decode projection for any weight type: lfm2_matmul_1x4_prequant_mt
 * (tools/lfm2_decode_1x4.c:795-813) through the CPU kernel table */
void ref_matmul_prequant_type(float *out, const void *w, uint32_t type, uint32_t n_rows, uint32_t n_cols,
                              const void *x_q8) {
    shim_state st;
    shim_save(&st);
    GGUFTensor t;
    memset(&t, 0, sizeof t);
    t.n_dims = 2;
    t.ne[0]  = n_cols;
    t.ne[1]  = n_rows;
    t.ne[2] = t.ne[3] = 1;
    t.type   = type;
    t.data   = w;
    const size_t per256 = type == GGML_TYPE_Q4_0 ? 8u * sizeof(block_q4_0_t)
                        : type == GGML_TYPE_Q8_0 ? 8u * sizeof(block_q8_0_t)
                        : type == GGML_TYPE_Q5_K ? sizeof(block_q5_K_t)
                        : type == GGML_TYPE_Q6_K ? sizeof(block_q6_K_t)
                        : type == GGML_TYPE_IQ4_XS ? sizeof(block_iq4_xs_t) : sizeof(block_q4_K_t);
    t.bytes = (size_t)n_rows * (n_cols / 256u) * per256;
    lfm2_matmul_1x4_prequant_mt(NULL, out, &t, NULL, (const block_q8_K_t *)x_q8);
    shim_restore(&st);
}

/* ---- CPU timing of the batched-prefill attention (baseline only) -------------- */
/* lfm2_forward_gqa_batch's per-row dispatch (tools/lfm2_prefill_batch.c:1074-1091):
 * GQAAttnTaskCtx + lfm2_gqa_heads_worker_task over the query heads, fp16
 * caches, for n_rows rows at positions pos[] with their q rows (fp32); the
 * pool is created once.  Returns the best of reps passes in seconds. */
double ref_time_prefill_rows(const float *q, const uint16_t *k16, const uint16_t *v16, const uint32_t *pos,
                             float *out, uint32_t n_rows, uint32_t n_head_q, uint32_t kv_mul, uint32_t kv_dim,
                             uint32_t max_seq, uint32_t n_threads, uint32_t reps, uint32_t *threads_out) {
    shim_state st;
    shim_save(&st);
    LFM2ThreadPool pool;
    lfm2_threadpool_init(&pool, n_threads);
    if (threads_out) *threads_out = pool.n_threads;
    float *att  = (float *)calloc((size_t)n_head_q * max_seq, sizeof(float));
    double best = 1e30;
    for (uint32_t r = 0; r < reps && att; ++r) {
        const double t0 = shim_now();
        for (uint32_t i = 0; i < n_rows; ++i) {
            GQAAttnTaskCtx ctx = {
                .pool = &pool, .q = q + (size_t)i * n_head_q * 64u, .k_cache = NULL, .v_cache = NULL,
                .k_cache_f16 = k16, .v_cache_f16 = v16, .att = att, .xb = out + (size_t)i * n_head_q * 64u,
                .n_head_q = n_head_q, .kv_mul = kv_mul, .head_dim = 64u, .kv_dim = kv_dim,
                .max_seq_len = max_seq, .pos = pos[i], .scale = 1.0f / sqrtf(64.0f)};
            lfm2_parallel_for(&pool, n_head_q, 1, lfm2_gqa_heads_worker_task, &ctx);
        }
        const double dt = shim_now() - t0;
        if (dt < best) best = dt;
    }
    free(att);
    lfm2_threadpool_free(&pool);
    shim_restore(&st);
    return best;
}
