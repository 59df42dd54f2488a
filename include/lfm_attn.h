/*
 * lfm_attn.h -- C-ABI of the MI355X (gfx950) attention path for the LFM2 /
 * LFM2.5 / LFM3 forward stacks.
 *
 * The reference engine (avisheksharmacoder/laii) has no FFI for attention:
 * each forward stack fills a task-context struct and calls
 * lfm2_parallel_for(pool, n_items, chunk, worker, &ctx).  Every lfm_hip_*
 * entry point below replaces one of those dispatches (cited per function) and
 * takes the same fields, minus the thread pool and the optional Q8_K output
 * (which stays with the caller, in front of the wo projection).
 *
 * Conventions
 *   - Pointers passed to lfm_hip_* are DEVICE pointers (hipMalloc'd, or from
 *     lfm_attn_dev_alloc).  Layouts are the reference's: KV caches are
 *     token-major uint16_t (IEEE binary16) [slot][n_head_kv][head_dim], Q and
 *     outputs are float [row][n_head_q][head_dim].
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and is asynchronous; lfm_attn_stream_sync() waits for it.
 *   - Every function returns LFM_ATTN_OK (0) or a negative status.  Invalid
 *     shapes and positions are rejected on the host before any launch; no
 *     partial work is enqueued for a rejected call.
 *   - Entry points that split the key range across workgroups use a
 *     library-owned device workspace (grown on demand, one per device):
 *     work on one device must run on one stream at a time, since two calls
 *     on different streams with no synchronization between them can overlap
 *     on the GPU and race on it (whether one host thread enqueued them or
 *     several).
 */
#ifndef LFM_ATTN_H
#define LFM_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ---------------------------------------------------------------- */
#define LFM_ATTN_OK            0
#define LFM_ATTN_E_INVALID    -1 /* null pointer, bad shape or geometry            */
#define LFM_ATTN_E_RANGE      -2 /* position outside the cache / window            */
#define LFM_ATTN_E_UNSUPPORTED -3 /* shape this build has no kernel for            */
#define LFM_ATTN_E_DEVICE     -4 /* HIP runtime error (see lfm_attn_last_error)    */
#define LFM_ATTN_E_NOMEM      -5 /* device allocation failed                       */
#define LFM_ATTN_E_IO         -6 /* a file could not be written                     */
#define LFM_ATTN_E_SCRATCH    -7 /* more split partials than the no-alloc scratch holds */

typedef void *lfm_attn_stream_t; /* hipStream_t */

const char *lfm_attn_status_string(int status);
/* Text of the last HIP error seen by this thread ("" if none). */
const char *lfm_attn_last_error(void);
/* Diagnostic, no reference counterpart: the form of this thread's last
 * decode / step attention launch -- "wg" (one workgroup per sequence and KV
 * head, in-workgroup merge), "grid" (fixed key chunks + merge kernel),
 * "balanced" (tile shares + merge kernel), "balanced-dma" (the same with
 * LDS-streamed segments) or "generic" ("" before any). */
const char *lfm_attn_last_plan(void);
const char *lfm_attn_version(void);

/* Tuning and tests, no reference counterpart: overrides of the launch
 * plans, process-wide.  Split-KV attention: plan NULL, "" or "auto" lets the
 * library choose; "grid", "balanced", "balanced-dma" (the balanced plan with
 * K and V streamed into per-wave LDS rings; head_dim 64, up to 32 query
 * columns, no fused prologue, else "balanced") or "wg" forces that form;
 * waves (1, 2, 4, 8), chunk (keys per workgroup) and min_tiles (32-key tiles
 * per balanced workgroup) force those counts.  prefill_chain: consecutive query tiles
 * per workgroup of a sliding-window lfm_hip_lfm3_prefill_f16.  0 =
 * automatic for every count.  The environment variables LFM_ATTN_PLAN,
 * LFM_ATTN_WAVES, LFM_ATTN_CHUNK, LFM_ATTN_MINTILES and
 * LFM_ATTN_PREFILL_CHAIN seed the overrides once, at the library's first
 * launch or first call of this function; launches never read the
 * environment.  Set it between launches, not while another thread
 * launches. */
int lfm_attn_set_tuning(const char *plan, uint32_t waves, uint32_t chunk, uint32_t min_tiles,
                        uint32_t prefill_chain);
/* Diagnostic, no reference counterpart, needs no device: the plan the
 * split-KV attention takes for a batch (n_seq sequences x n_rows rows, head
 * shape, sliding window, keys_hint as lfm_hip_gqa_f16_varlen; positions on
 * the device or one host position; fused = the step entry's prologue) on a
 * device of n_cus compute units under the current overrides: *plan = "wg",
 * "grid", "balanced", "balanced-dma" or "generic" (no split-KV kernel for
 * the shape);
 * out3 = {waves per workgroup, grid key splits, grid chunk} (0 where the
 * plan has none). */
int lfm_attn_plan_preview(uint32_t n_seq, uint32_t n_rows, uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                          uint32_t window_len, uint32_t keys_hint, int positions_on_device, int fused, uint32_t n_cus,
                          const char **plan, uint32_t out3[3]);

/* Diagnostic, no reference counterpart, needs no device: the launch shape
 * lfm_hip_lfm3_prefill_f16 takes for a prompt (n_seq x n_tok rows from
 * position pos_0, sliding window or 0, head shape) under the current
 * overrides: out4 = {query positions per tile, tiles per workgroup, short
 * tiles at the sequence start dispatched first (their window reaches before
 * position 0), workgroups}.  LFM_ATTN_E_UNSUPPORTED for a head shape that
 * entry point does not take. */
int lfm_attn_prefill_plan_preview(uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint32_t window_len,
                                  uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim, uint32_t out4[4]);

/* ---- device plumbing (so C11 callers need no HIP headers) ------------------ */
int lfm_attn_device_count(int *count);
/* Makes `device` current for this thread and resolves the device address of
 * its no-alloc scratch (lfm_hip_gqa_f16_varlen_noalloc), which loads the
 * library's code object there if it is not yet loaded. */
int lfm_attn_set_device(int device);
int lfm_attn_dev_alloc(void **ptr, size_t bytes);
int lfm_attn_dev_free(void *ptr);
int lfm_attn_copy_h2d(void *dst_dev, const void *src_host, size_t bytes, lfm_attn_stream_t stream);
int lfm_attn_copy_d2h(void *dst_host, const void *src_dev, size_t bytes, lfm_attn_stream_t stream);
int lfm_attn_copy_d2d(void *dst_dev, const void *src_dev, size_t bytes, lfm_attn_stream_t stream);
int lfm_attn_memset(void *dst_dev, int value, size_t bytes, lfm_attn_stream_t stream);
int lfm_attn_stream_sync(lfm_attn_stream_t stream);

/* Observability: while set (per host thread), every attention call records
 * `before` / `after` (hipEvent_t handles) on its stream immediately around its
 * main attention kernel, excluding the split merge; hipEventElapsedTime of the
 * pair is that kernel's duration.  NULL, NULL switches it off. */
int lfm_attn_profile_events(void *before, void *after);

/* ---- index math (host copy of what the kernels compute) -------------------- */
/* Row plan of tools/lfm3_engine.c:862-873:
 * out5 = {t_start, count, seg1_slot, seg1_len, seg2_len}. */
int lfm_attn_seg_plan(uint32_t abs_pos, uint32_t window_len, uint32_t cap, uint32_t out5[5]);
/* Slot holding absolute position p: p % cap with a window, p without. */
uint32_t lfm_attn_slot_of(uint32_t p, uint32_t window_len, uint32_t cap);

/* ---- RoPE tables (host, double-precision angles; bit-identical) ------------- */
/* Replaces lfm2_rope_lut_init, tools/lfm2_kernels_fast.c:370-388.
 * cos_lut/sin_lut: HOST float[max_seq][head_dim/2]. */
int lfm_attn_rope_lut_lfm2(float *cos_lut, float *sin_lut, uint32_t max_seq, uint32_t head_dim,
                           float freq_base);
/* Replaces lfm3_rope_lut_init, tools/lfm3_engine.c:403-450 (partial RoPE:
 * identity pairs for i >= rope_dim/2 and for rope_freqs[i] >= 1e10 or <= 0). */
int lfm_attn_rope_lut_lfm3(float *cos_lut, float *sin_lut, uint32_t max_seq, uint32_t head_dim,
                           uint32_t rope_dim, float freq_base, const float *rope_freqs,
                           uint32_t n_rope_freqs);

/* Replaces the float-angle table of the production LFM2 stacks, built by
 * lfm2_state_init (tools/lfm2_forward.c:572-581) and lfm2_batch_state_init
 * (tools/lfm2_prefill_batch.c:727-736): freq_i = powf(base, -(2i / head_dim))
 * in float, entries cosf / sinf of the float product (float)p * freq_i
 * (freq_base <= 0 means 10000).  The table of LFM_PROLOGUE_TABLE.
 * cos_tab/sin_tab: HOST float[max_seq][head_dim/2]. */
int lfm_attn_rope_table_lfm2(float *cos_tab, float *sin_tab, uint32_t max_seq, uint32_t head_dim,
                             float freq_base);

/* Gen-1 RoPE row (host): cos_row[i], sin_row[i] of (float)pos * (1 /
 * powf(theta, 2i / head_dim)), i < head_dim / 2, computed in float with
 * powf/cosf/sinf on every call as lfm_rope_neox does (src/lfm_forward.c:97-111;
 * the Gen-1 engine has no table).  Upload the row for the position of a
 * lfm_hip_gen1_gqa_step call. */
int lfm_attn_rope_row_gen1(float *cos_row, float *sin_row, uint32_t head_dim, uint32_t pos, float theta);

/* ---- prologue: per-head QK-RMSNorm + NeoX RoPE (+ RNE fp16 KV store) -------- */
/* Prologue forms.  The reference runs two LFM2 prologues that differ in their
 * RoPE table (an input here: cos_lut/sin_lut) and in the order in which
 * RMSNorm adds the squares; rows match the chosen one bit for bit.
 *   LFM_PROLOGUE_FAST   lfm2_qk_norm_rope_avx2 (tools/lfm2_kernels_fast.c:403-497),
 *                       lfm3_qk_norm_rope_128_avx2 (tools/lfm3_engine.c:463-525):
 *                       the fast decode context and LFM3.  Tables:
 *                       lfm_attn_rope_lut_lfm2 / lfm_attn_rope_lut_lfm3.
 *   LFM_PROLOGUE_TABLE  lfm2_qk_norm_and_rope (tools/lfm2_forward.c:775-830) and
 *                       lfm2_qk_norm_and_rope_table (tools/lfm2_prefill_batch.c:
 *                       826-893): the lfm2_forward.c decode, speculative verify
 *                       and prompt prefill.  lfm2_rmsnorm's order
 *                       (tools/lfm2_forward.c:669-684): eight fma chains over
 *                       dims 8k + j, added in double.  Table:
 *                       lfm_attn_rope_table_lfm2.
 * Any other value returns LFM_ATTN_E_INVALID. */
#define LFM_PROLOGUE_FAST  0
#define LFM_PROLOGUE_TABLE 1

/* Replaces lfm2_qk_norm_rope_simd (tools/lfm2_kernels_fast.c:403-497, :511-547),
 * lfm3_qk_norm_rope_simd (tools/lfm3_engine.c:463-525, :599-666) and, with
 * LFM_PROLOGUE_TABLE, lfm2_qk_norm_and_rope_table / lfm2_qk_norm_and_rope.
 * vec: [n_heads][head_dim] float.  norm_w: [head_dim] or NULL (no norm).
 * cos_lut/sin_lut: DEVICE [>= pos+1][head_dim/2].  With dst_f16 != NULL the
 * rotated heads are stored there as RNE fp16 and vec is not modified;
 * otherwise vec is rotated in place.  head_dim even, <= 256. */
int lfm_hip_qk_norm_rope(float *vec, uint16_t *dst_f16, uint32_t n_heads, uint32_t head_dim,
                         const float *norm_w, float eps, const float *cos_lut,
                         const float *sin_lut, uint32_t pos, int prologue, lfm_attn_stream_t stream);

/* Replaces lfm2_store_fp32_to_fp16_simd (tools/lfm2_kernels_fast.c:500-507,
 * :549-555) and lfm3_store_f32_to_f16 (tools/lfm3_engine.c:133-153): RNE. */
int lfm_hip_store_fp32_to_fp16(uint16_t *dst_f16, const float *src, uint32_t n,
                               lfm_attn_stream_t stream);

/* Batched prologue for n_seq sequences x n_rows consecutive tokens (row r of
 * sequence s is position pos_0[s] + r): Q rotated in place, K rotated and
 * stored as RNE fp16 at slot lfm_attn_slot_of(pos, window_len, cap), V stored
 * as RNE fp16 at the same slot.  This is the per-token prologue of
 * lfm2_forward_gqa_batch (tools/lfm2_prefill_batch.c:1029-1072) and
 * lfm3_forward_batch_core (tools/lfm3_engine.c:2006-2016) over many sequences.
 * q: [n_seq][n_rows][n_head_q][hd]; k, v: [n_seq][n_rows][n_head_kv][hd];
 * k_seq/v_seq: DEVICE arrays of n_seq DEVICE cache pointers; pos_0: DEVICE
 * uint32_t[n_seq]; prologue: LFM_PROLOGUE_FAST or LFM_PROLOGUE_TABLE. */
int lfm_hip_qkv_prologue(float *q, const float *k, const float *v, uint16_t *const *k_seq,
                         uint16_t *const *v_seq, const uint32_t *pos_0, uint32_t n_seq,
                         uint32_t n_rows, uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                         const float *q_norm_w, const float *k_norm_w, float eps,
                         const float *cos_lut, const float *sin_lut, uint32_t window_len,
                         uint32_t cap, int prologue, lfm_attn_stream_t stream);

/* ---- projections beside the attention path ------------------------------- */
/* Blocks are the reference's packed GGUF layouts (tools/lfm2_cpuid_quants.c:76-127):
 * block_q8_K 292 B (float d, int8 qs[256], int16 bsums[16]); block_q4_K 144 B
 * (fp16 d, fp16 dmin, uint8 scales[12], uint8 qs[128]).  n_cols % 256 == 0
 * (else LFM_ATTN_E_UNSUPPORTED). */

/* Q8_K quantization of n_rows rows of n_cols floats into y_q8_K
 * [n_rows][n_cols/256] blocks, bit-identical to the engine's AVX2 quantizer:
 * replaces lfm2_quantize_batch_q8_K_avx2 (tools/lfm2_prefill_batch.c:93-105)
 * and lfm2_quantize_row_q8_K_avx2 (tools/lfm2_cpuid_quants.c:585-635), and
 * the Q8_K output side effect of A1 (tools/lfm2_kernels_fast.c:804-807):
 * quantizing xb_out as one row of n_head_q * 64 floats gives the same blocks
 * as the per-4-head slices.  x 4-byte aligned; y 4-byte aligned. */
int lfm_hip_quantize_q8_K(const float *x, void *y_q8_K, uint32_t n_rows, uint32_t n_cols,
                          lfm_attn_stream_t stream);

/* Weight types of the projections (GGML ids; blocks as in
 * tools/lfm2_cpuid_quants.c:55-127, include/lfm2_simd_avx2.h:120-158), the
 * alignment a matrix needs, and the reference dot each row equals bit for bit:
 *   2  Q4_0   18 B / 32 weights (fp16 d, qs[16])             2  lfm2_vec_dot_q4_0_q8_K_avx2
 *   8  Q8_0   34 B / 32 weights (fp16 d, int8 qs[32])        2  lfm2_vec_dot_q8_0_q8_K_avx2
 *   12 Q4_K  144 B / 256 (d, dmin, scales[12], qs[128])     16  lfm2_vec_dot_q4_K_q8_K_avx2
 *   13 Q5_K  176 B / 256 (d, dmin, scales[12], qh[32], qs) 16  lfm2_vec_dot_q5_K_q8_K_avx2
 *   14 Q6_K  210 B / 256 (ql[128], qh[64], scales[16], d)    2  lfm2_vec_dot_q6_K_q8_K_avx2
 *   23 IQ4_XS 136 B / 256 (d, scales_h, scales_l[4], qs)     8  lfm2_vec_dot_iq4_xs_q8_K_avx2
 * n_cols must be a multiple of 256 (the Q8_K activations'). */
#define LFM_Q_TYPES {2u, 8u, 12u, 13u, 14u, 23u}

/* out[t][r] = (row r of the Q4_K matrix w_q4_K [n_rows][n_cols/256]) .
 * (token t of x_q8_K [n_tokens][n_cols/256]), bit-identical to
 * lfm2_vec_dot_q4_K_q8_K_avx2 (include/lfm2_simd_avx2.h:364-412) per row.
 * Replaces lfm2_matmul_1x4_prequant_mt (tools/lfm2_decode_1x4.c:795-813,
 * n_tokens = 1, e.g. the `wo` projection of x_q8 from attention) and the Q4_K
 * branch of lfm2_matmul_batch_avx2_mt (tools/lfm2_prefill_batch.c:479-510,
 * 598-634) after its quantize step.  w 16-byte aligned; x_q8_K and out
 * 4-byte aligned. */
int lfm_hip_matmul_q4_K(float *out, const void *w_q4_K, uint32_t n_rows, uint32_t n_cols,
                        const void *x_q8_K, uint32_t n_tokens, lfm_attn_stream_t stream);

/* Fused projections of one Q8_K activation set x_q8_K [n_tokens][n_cols/256]
 * through the Q, K, V and (optional) gate matrices in one pass: q_out[t][r] =
 * row r of wq . token t, likewise k, v, g.  Replaces
 * lfm2_gqa_qkv_fused_1x4_mt (tools/lfm2_decode_1x4.c:885-930; g_out NULL)
 * and lfm3_gqa_qkvg_1x4_mt (tools/lfm3_engine.c:1545-1598).  types[4] holds
 * each matrix's GGML type (LFM_Q_TYPES below); any other type gives
 * LFM_ATTN_E_UNSUPPORTED.  Each row is bit-identical to the reference's AVX2
 * 1x1 dot of its type.  The gate output is the raw projection: the attention
 * entry points take it as logits (gate_is_logit), which applies the
 * reference's sigmoid. */
/* out[t][r] = (row r of w, GGML type w_type, [n_rows][n_cols]) . (token t of
 * x_q8_K): lfm2_matmul_1x4_prequant_mt (tools/lfm2_decode_1x4.c:795-813) for
 * every weight type its kernel table serves (tools/lfm2_decode_1x4.c:597-690),
 * and those branches of lfm2_matmul_batch_avx2_mt after its quantize step.
 * Types and alignment as LFM_Q_TYPES; out and x_q8_K 4-byte aligned. */
int lfm_hip_matmul_prequant(float *out, const void *w, uint32_t w_type, uint32_t n_rows, uint32_t n_cols,
                            const void *x_q8_K, uint32_t n_tokens, lfm_attn_stream_t stream);

int lfm_hip_gqa_qkv_fused(float *q_out, float *k_out, float *v_out, float *g_out, const void *wq,
                          const void *wk, const void *wv, const void *wg, const uint32_t types[4],
                          uint32_t q_rows, uint32_t k_rows, uint32_t v_rows, uint32_t g_rows,
                          uint32_t n_cols, const void *x_q8_K, uint32_t n_tokens,
                          lfm_attn_stream_t stream);

/* ---- attention ------------------------------------------------------------ */
/* A1 -- replaces OnlineGQATaskCtx + lfm2_parallel_for(pool, ceil(n_head_q/4), 1,
 * lfm2_online_gqa_f16_worker_simd, &ctx), tools/lfm2_kernels_fast.c:685-697,
 * 700-872, 1052-1066.  head_dim 64; kv_h = h / kv_mul; keys [0, pos].
 * q, xb_out: [n_head_q][64] float; caches [>= pos+1][kv_dim] fp16. */
int lfm_hip_online_gqa_f16(const float *q, const uint16_t *k_cache_f16,
                           const uint16_t *v_cache_f16, float *xb_out, uint32_t n_head_q,
                           uint32_t kv_mul, uint32_t kv_dim, uint32_t pos, float scale,
                           lfm_attn_stream_t stream);

/* A2 -- replaces GQAAttnTaskCtx + lfm2_parallel_for(pool, n_head_q, 1,
 * lfm2_gqa_heads_worker_task, &ctx), tools/lfm2_threadpool.c:745-931, as called
 * at tools/lfm2_prefill_batch.c:1074-1091 and tools/lfm2_forward.c:1018-1035.
 * With both f16 caches non-NULL: FP16 online branch (only the first 64 output
 * dims are written when head_dim > 64, as the reference does).  Otherwise the
 * FP32 caches k_cache/v_cache ([max_seq_len][kv_dim] float) are used.
 * head_dim % 8 == 0, head_dim <= 256. */
int lfm_hip_gqa_heads(const float *q, const float *k_cache, const float *v_cache,
                      const uint16_t *k_cache_f16, const uint16_t *v_cache_f16, float *xb,
                      uint32_t n_head_q, uint32_t kv_mul, uint32_t head_dim, uint32_t kv_dim,
                      uint32_t max_seq_len, uint32_t pos, float scale, lfm_attn_stream_t stream);

/* A6 -- replaces steps 2-4 of the Gen-1 lfm_gqa_step (src/lfm_forward.c:
 * 184-244, include/lfm_forward.h:64-72): per head RMSNorm
 * (lfm_vec_rmsnorm_f32, src/lfm_simd.c:125-174) and NeoX RoPE of q and k,
 * the FP32 append of k and v at cache row pos, then softmax(q.k / sqrt(hd)).v
 * over rows 0..pos of every query head (kv head = h / (n_heads_q /
 * n_heads_kv)).  q, k, v: the projections ([n_heads][head_dim] float, device);
 * q is normalised and rotated in place (the reference's arena scratch).
 * q_norm, k_norm: [head_dim] or NULL (no weight).  k_cache, v_cache:
 * [max_seq][n_heads_kv * head_dim] float.  cos_row, sin_row: the row of
 * lfm_attn_rope_row_gen1 for pos (device).  attn_out: [n_heads_q][head_dim];
 * the wo projection stays with the caller.  head_dim % 8 == 0, <= 256. */
int lfm_hip_gen1_gqa_step(float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                          float *k_cache, float *v_cache, float *attn_out, uint32_t pos, uint32_t max_seq,
                          uint32_t n_heads_q, uint32_t n_heads_kv, uint32_t head_dim, float eps,
                          const float *cos_row, const float *sin_row, lfm_attn_stream_t stream);

/* A3 -- replaces lfm3_online_gqa_f16_dispatch, tools/lfm3_engine.c:1155-1204
 * (workers :851-946, :1057-1153).  Row b is position pos_0 + b and attends
 * the plan of lfm_attn_seg_plan(pos_0 + b, window_len, swa_cap); output is
 * o * (gate_sig[b][h] / l) (gate 1 when gate_sig is NULL).
 * q_batch, xb_out: [B][n_head_q][head_dim]; gate_sig: [B][n_head_q] or NULL. */
int lfm_hip_lfm3_online_gqa_f16_dispatch(const float *q_batch, const float *gate_sig,
                                         const uint16_t *k_cache_f16,
                                         const uint16_t *v_cache_f16, float *xb_out, uint32_t B,
                                         uint32_t pos_0, uint32_t window_len, uint32_t swa_cap,
                                         uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                                         lfm_attn_stream_t stream);

/* Multi-sequence form of A1/A2/A3 (decode batches and the B<=8 speculative
 * verify of tools/lfm2_speculative_pld.c:388-461 over many sequences): n_seq
 * independent caches, n_rows consecutive query rows per sequence; row r of
 * sequence s is position pos_0[s] + r and attends
 * lfm_attn_seg_plan(pos_0[s] + r, window_len, cap) of its own cache.
 * q, out: [n_seq][n_rows][n_head_q][head_dim] float.
 * gate: [n_seq][n_rows][n_head_q] float or NULL; sigmoid is applied in the
 *   epilogue when gate_is_logit != 0 (tools/lfm3_engine.c:1588-1597), the
 *   values are used as-is otherwise.
 * k_seq, v_seq: DEVICE arrays of n_seq DEVICE cache pointers; pos_0: DEVICE
 *   uint32_t[n_seq].
 * keys_hint: upper bound of the keys a row attends (the engine knows its
 *   positions); it sizes the key split (0 = unknown).  Rows attending more
 *   keys are still handled correctly, with longer chunks.
 * scale: multiplies q.k (1/sqrtf(head_dim) in every reference caller). */
int lfm_hip_gqa_f16_varlen(const float *q, const float *gate, int gate_is_logit,
                           const uint16_t *const *k_seq, const uint16_t *const *v_seq,
                           const uint32_t *pos_0, float *out, uint32_t n_seq, uint32_t n_rows,
                           uint32_t keys_hint, uint32_t n_head_q, uint32_t n_head_kv,
                           uint32_t head_dim, uint32_t window_len, uint32_t cap, float scale,
                           lfm_attn_stream_t stream);

/* One attention step of the forward stacks with the prologue fused into the
 * attention kernel: per row, QK-RMSNorm + NeoX RoPE of the raw query and of
 * the raw new-token key, the RNE fp16 store of that key and value at the
 * position's slot, then attention over the row's keys (times the gate).
 * Replaces steps 3-4 of lfm2_forward_gqa_fast (tools/lfm2_kernels_fast.c:
 * 1046-1066: lfm2_qk_norm_rope_simd, the fp16 stores, then the
 * OnlineGQATaskCtx dispatch), the per-token prologue + attention of
 * lfm2_forward_gqa_batch (tools/lfm2_prefill_batch.c:1029-1092) and the
 * attention block of lfm3_forward_token_internal / lfm3_forward_batch_core
 * (tools/lfm3_engine.c:1885-1896, 2006-2022), over many sequences.
 * q: raw queries [n_seq][n_rows][n_head_q][head_dim] (left unchanged);
 * k, v: raw new-token rows [n_seq][n_rows][n_head_kv][head_dim];
 * q_norm_w, k_norm_w: [head_dim] or NULL (no norm); cos_lut/sin_lut: the RoPE
 * table [> last position][head_dim / 2]; prologue: LFM_PROLOGUE_FAST (the
 * lfm2_kernels_fast.c and LFM3 stacks) or LFM_PROLOGUE_TABLE (lfm2_forward.c
 * and lfm2_prefill_batch.c, with the table of lfm_attn_rope_table_lfm2); the
 * rest as lfm_hip_gqa_f16_varlen.
 * With a sliding window, window_len + n_rows - 1 <= cap (each row's window
 * survives the later rows' ring writes).  Head dims 64 and 128 run one
 * attention launch (plus the split merge where the keys are split); other
 * head dims run the prologue on a copy of q and the generic kernel. */
int lfm_hip_gqa_f16_step(const float *q, const float *k, const float *v, const float *gate, int gate_is_logit,
                         uint16_t *const *k_seq, uint16_t *const *v_seq, const uint32_t *pos_0, float *out,
                         uint32_t n_seq, uint32_t n_rows, uint32_t keys_hint, uint32_t n_head_q,
                         uint32_t n_head_kv, uint32_t head_dim, uint32_t window_len, uint32_t cap, float scale,
                         const float *q_norm_w, const float *k_norm_w, float eps, const float *cos_lut,
                         const float *sin_lut, int prologue, lfm_attn_stream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): lfm_hip_gqa_f16_varlen with the same arguments, kernels
 * and results, whose split partials go to a fixed device array of the
 * library (LFM_ATTN_NOALLOC_SCRATCH_BYTES per device, held until the process
 * ends) instead of the growing workspace, so the call allocates nothing.  A
 * batch whose partials need more returns LFM_ATTN_E_SCRATCH before anything
 * is launched.  Every call on a device shares that device's array: calls that
 * overlap on one device (any streams) race.  Nothing in the array needs to
 * start at zero: every partial the merge reads is written earlier by the
 * same call.  The array's device address is looked up once per device, by
 * lfm_attn_set_device or else by the first call of this function there:
 * call one of them on each device before capturing a graph that contains
 * this call, since the lookup may load the library's code object. */
#define LFM_ATTN_NOALLOC_SCRATCH_BYTES (32u << 20)
int lfm_hip_gqa_f16_varlen_noalloc(const float *q, const float *gate, int gate_is_logit,
                                   const uint16_t *const *k_seq, const uint16_t *const *v_seq,
                                   const uint32_t *pos_0, float *out, uint32_t n_seq, uint32_t n_rows,
                                   uint32_t keys_hint, uint32_t n_head_q, uint32_t n_head_kv,
                                   uint32_t head_dim, uint32_t window_len, uint32_t cap, float scale,
                                   lfm_attn_stream_t stream);

/* Causal prefill on MFMA -- the prompt path of lfm2_prefill_prompt /
 * lfm2_forward_batch (tools/lfm2_prefill_batch.c:1129-1199), whose attention
 * runs lfm2_gqa_heads_worker_task once per row (:1029-1092).  Row i of
 * sequence s is position pos_0 + i and attends keys [0, pos_0 + i] of that
 * sequence's cache, which must already hold rows 0 .. pos_0 + n_tok - 1.
 * q:   [n_seq][n_tok][n_head_q][head_dim] float (RoPE applied), as the
 *      reference's rows; q * scale * log2(e) enters the MFMA as fp16.
 * k,v: sequence s at k + s * kv_seq_stride elements, [slot][n_head_kv][head_dim].
 * out: [n_seq][n_tok][n_head_q][head_dim] float.
 * head_dim 64 (MFMA kernel); other head dims return LFM_ATTN_E_UNSUPPORTED
 * (the reference's fp16 LFM2 heads worker writes at most 64 output dims per
 * head, tools/lfm2_threadpool.c:778-828; LFM3 layers of head_dim 128 use
 * lfm_hip_lfm3_prefill_f16).  Softmax and accumulation are fp32; P enters
 * the P.V product as fp16. */
int lfm_hip_prefill_f16(const float *q, const uint16_t *k, const uint16_t *v, float *out,
                        uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint64_t kv_seq_stride,
                        uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim, float scale,
                        lfm_attn_stream_t stream);

/* Causal prefill of an LFM3 attention layer (full or sliding-window, with the
 * output gate) on MFMA: the attention of lfm3_forward_batch_core
 * (tools/lfm3_engine.c:1918-2055; per-row window :862-873, gate scaling
 * :902-911), whose batches hold at most LFM2_MAX_BATCH rows, for a whole
 * prompt in one launch.  Row i of sequence s is position p = pos_0 + i and
 * attends keys [t_start(p), p], t_start(p) = p + 1 - window_len when
 * window_len > 0 and p + 1 > window_len, else 0; with gate non-NULL
 * ([n_seq][n_tok][n_head_q]) its output is scaled by sigmoid(gate) when
 * gate_is_logit, else by gate.
 * K/V row r of sequence s (at k + s * kv_seq_stride elements,
 * [row][n_head_kv][head_dim]) holds position kv_pos0 + r, for positions
 * kv_pos0 .. pos_0 + n_tok - 1: a full layer passes its cache (kv_pos0 = 0);
 * a sliding-window layer passes a linear copy of the window before the
 * prompt plus the prompt's rows (a ring of window + 8 slots cannot hold a
 * whole prompt).  kv_pos0 must not exceed t_start(pos_0)
 * (LFM_ATTN_E_INVALID).  q, out as for lfm_hip_prefill_f16.  head_dim 128
 * (LFM3) or 64, with n_head_q / n_head_kv dividing 128, else
 * LFM_ATTN_E_UNSUPPORTED. */
int lfm_hip_lfm3_prefill_f16(const float *q, const uint16_t *k, const uint16_t *v, const float *gate,
                             int gate_is_logit, float *out, uint32_t n_seq, uint32_t n_tok, uint32_t pos_0,
                             uint32_t kv_pos0, uint64_t kv_seq_stride, uint32_t window_len, uint32_t n_head_q,
                             uint32_t n_head_kv, uint32_t head_dim, float scale, lfm_attn_stream_t stream);

/* ---- attention-sink eviction on device caches ------------------------------ */
/* When the position nears max_seq the engine keeps the first n_sink rows,
 * drops the next n_discard and moves the remaining n_keep = pos - n_sink -
 * n_discard rows down to n_sink, counter-rotating every moved key by
 * -n_discard positions with the RoPE table row of position n_discard
 * (trigger: src/lfm2_api.c:871-891).  On return *inout_pos is the new
 * position n_sink + n_keep.  Like the reference, nothing moves and
 * *inout_pos stays when n_discard == 0 or *inout_pos <= n_sink + n_discard.
 * Key pairs (i, i + head_dim/2) rotate as fma(lo, c, hi*s) and
 * fma(hi, c, -(lo*s)) in fp32 with an RNE fp16 store, bit-identical to the
 * reference's AVX2 kernels; values move unchanged.  Asynchronous on `stream`.
 *
 * LFM2 -- lfm2_kv_cache_shift_sinks (tools/lfm2_runtime_features.c:744-833,
 * dispatcher :984-1001).  k_caches / v_caches: host arrays of n_layers device
 * cache pointers ([max_seq][n_head_kv[l]][head_dim] fp16); a layer with a NULL
 * cache or n_head_kv[l] == 0 (a ShortConv layer) is skipped.  cos_lut /
 * sin_lut: the device LFM2 table ([lut_rows][head_dim/2], as built by
 * lfm_attn_rope_lut_lfm2).  head_dim != 64 leaves everything unchanged, as
 * the reference does.  Returns LFM_ATTN_E_RANGE when n_discard >= lut_rows. */
int lfm_hip_kv_cache_shift_sinks(uint16_t *const *k_caches, uint16_t *const *v_caches,
                                 uint32_t n_layers, const uint32_t *n_head_kv, uint32_t head_dim,
                                 const float *cos_lut, const float *sin_lut, uint32_t lut_rows,
                                 uint32_t *inout_pos, uint32_t n_sink, uint32_t n_discard,
                                 lfm_attn_stream_t stream);
/* LFM3 -- lfm3_kv_cache_shift_sinks (tools/lfm2_runtime_features.c:1055-1163).
 * layer_kind[l]: 0 skipped (ShortConv), 1 full attention (linear cache,
 * shifted like LFM2 with the full table), 2 sliding window (ring of swa_cap
 * slots, 0 = window + 8; window = sliding_window, 0 = 256): the last
 * min(new_pos, window) positions are re-slotted at their new positions, the
 * kept ones counter-rotated with the SWA table.  The re-slotting goes through
 * the library's device workspace.  Like the reference, nothing moves when
 * n_discard is not below both table row counts or head_dim is odd. */
int lfm_hip_lfm3_kv_cache_shift_sinks(uint16_t *const *k_caches, uint16_t *const *v_caches,
                                      uint32_t n_layers, const uint32_t *n_head_kv,
                                      const uint8_t *layer_kind, uint32_t head_dim,
                                      const float *cos_full, const float *sin_full,
                                      uint32_t full_rows, const float *cos_swa,
                                      const float *sin_swa, uint32_t swa_rows,
                                      uint32_t sliding_window, uint32_t swa_cap,
                                      uint32_t *inout_pos, uint32_t n_sink, uint32_t n_discard,
                                      lfm_attn_stream_t stream);

/* ---- engine context: device-resident KV + host-pointer calls (C11) -------- */
/* The forward stacks own their KV caches in host memory
 * (tools/lfm2_forward.c:612-622, tools/lfm3_engine.c:1740-1769).  A GPU
 * drop-in keeps them in HBM instead: the context owns one fp16 K and V cache
 * per attention layer (same token-major layout), the RoPE tables and the
 * QK-norm weights, and each call moves only Q/K/V/gate in and the attention
 * output out.  Calls are synchronous (the output is in host memory on
 * return), like the pool dispatch they replace; a context is not thread-safe. */
typedef struct lfm_attn_ctx lfm_attn_ctx;

typedef struct {
    uint32_t n_layers;        /* attention layers held by the context              */
    uint32_t n_head_q;
    uint32_t n_head_kv;
    uint32_t head_dim;
    uint32_t max_seq;         /* positions (LUT rows, linear cache slots)          */
    uint32_t sliding_window;  /* SWA window (LFM3), 0 when no layer uses one       */
    uint32_t swa_cap;         /* ring slots of SWA layers (engine: window + 8)     */
    const uint8_t *layer_is_swa; /* [n_layers] or NULL (no SWA layer)             */
    float eps;                /* QK RMSNorm epsilon                                */
    float rope_base;          /* full / LFM2 layers                                */
    float rope_base_swa;      /* SWA layers (LFM3: 1e4)                            */
    uint32_t rope_dim;        /* LFM3 partial RoPE (0 = head_dim)                  */
    const float *rope_freqs;  /* LFM3 rope_freqs factors or NULL                   */
    uint32_t n_rope_freqs;
    int lfm3;                 /* 1: LFM3 tables (lfm3_rope_lut_init), 0: LFM2      */
    int prologue;             /* LFM2 only: LFM_PROLOGUE_FAST (lfm2_kernels_fast.c,
                                 table lfm2_rope_lut_init) or LFM_PROLOGUE_TABLE
                                 (lfm2_forward.c / lfm2_prefill_batch.c, their
                                 float-angle table); LFM3 takes FAST only.  Sink
                                 eviction counter-rotates with the
                                 lfm2_rope_lut_init table either way, as
                                 src/lfm2_api.c:883-888 does                      */
} lfm_attn_geom;

int lfm_attn_ctx_create(lfm_attn_ctx **out, const lfm_attn_geom *geom);
void lfm_attn_ctx_destroy(lfm_attn_ctx *ctx);
/* Per-layer QK-RMSNorm weights ([head_dim] host floats, NULL = no norm). */
int lfm_attn_ctx_set_norms(lfm_attn_ctx *ctx, uint32_t layer, const float *q_norm_w,
                           const float *k_norm_w);

/* One attention step of `layer` for B consecutive positions pos_0 .. pos_0+B-1
 * (B = 1 decode; B <= 8 prompt chunk or speculative verify):
 *   QK-RMSNorm + RoPE of q and k, RNE fp16 store of k and v at each position's
 *   slot, then attention of row b over its window, times sigmoid(gate) when
 *   gate_logits is non-NULL.
 * Replaces steps 3-4 of lfm2_forward_gqa_fast (tools/lfm2_kernels_fast.c:1046-1066),
 * the per-token loop of lfm2_forward_gqa_batch (tools/lfm2_prefill_batch.c:1029-1092)
 * and the attention block of lfm3_forward_token_internal / lfm3_forward_batch_core
 * (tools/lfm3_engine.c:1885-1896, 2006-2022).
 * q: [B][n_head_q][head_dim], k, v: [B][n_head_kv][head_dim], gate_logits:
 * [B][n_head_q] or NULL, out: [B][n_head_q][head_dim] -- all HOST floats.
 * Returns LFM_ATTN_E_RANGE when pos_0 + B > max_seq. */
int lfm_attn_ctx_forward(lfm_attn_ctx *ctx, uint32_t layer, uint32_t pos_0, uint32_t B,
                         const float *q, const float *k, const float *v,
                         const float *gate_logits, float *out);

/* Copy `n_slots` cache rows of a layer starting at `slot` between the device
 * cache and host memory (fp16 bits, [slot][n_head_kv][head_dim]) -- the data
 * a checkpoint or .lfmcache file stores (tools/lfm2_moe_checkpoint.c:472-560,
 * tools/lfm2_sys_cache.c:504-799).  Round trips are bit-exact. */
/* Prompt prefill of one attention layer: n_rows tokens at positions
 * pos_0 .. pos_0 + n_rows - 1, q/k/v/gate/out as in lfm_attn_ctx_forward
 * with n_rows rows (any count).  lfm2_forward_batch runs a prompt through
 * the layer LFM2_MAX_BATCH tokens at a time (tools/lfm2_prefill_batch.c:
 * 1129-1199, attention :1029-1092); here a full-attention layer of head_dim
 * 64 without a gate takes the whole prompt in one MFMA prefill (prologue,
 * then every row attends keys 0 .. its position), and other layers run the
 * step over chunks of 8 rows.  Synchronous; LFM_ATTN_E_RANGE past max_seq. */
int lfm_attn_ctx_prefill(lfm_attn_ctx *ctx, uint32_t layer, uint32_t pos_0, uint32_t n_rows,
                         const float *q, const float *k, const float *v, const float *gate_logits,
                         float *out);

int lfm_attn_ctx_kv_export(lfm_attn_ctx *ctx, uint32_t layer, uint32_t slot, uint32_t n_slots,
                           uint16_t *k_host, uint16_t *v_host);
int lfm_attn_ctx_kv_import(lfm_attn_ctx *ctx, uint32_t layer, uint32_t slot, uint32_t n_slots,
                           const uint16_t *k_host, const uint16_t *v_host);
/* Attention-sink eviction over every layer of the context (LFM2: head_dim 64
 * only, as the reference; LFM3: full and SWA layers), with the context's own
 * tables; synchronous.  Same semantics as lfm_hip_kv_cache_shift_sinks /
 * lfm_hip_lfm3_kv_cache_shift_sinks. */
int lfm_attn_ctx_shift_sinks(lfm_attn_ctx *ctx, uint32_t *inout_pos, uint32_t n_sink,
                             uint32_t n_discard);
/* FNV-1a 64 of n_bytes of device memory (16-byte aligned), continuing from
 * h_in (the offset basis 14695981039346656037 for a fresh hash): the value
 * lfm2_fnv1a_update (tools/lfm2_sys_cache.c:382-389) returns for the same
 * bytes, computed in parallel on the device.  Synchronous: *h_out is set on
 * return.  n_bytes == 0 returns h_in. */
int lfm_hip_fnv1a64(const void *data, size_t n_bytes, uint64_t h_in, uint64_t *h_out,
                    lfm_attn_stream_t stream);

/* ---- prompt cache files (.lfmcache v1) ----------------------------------------
 * The engine's disk-backed prompt cache (tools/lfm2_sys_cache.c:354-799):
 * a 64-byte header (magic "01LFM2PC", version 1, token count, model
 * fingerprint, layer count, n_embd, n_head_q, ShortConv cache length, payload
 * bytes), the token ids, then per model layer either the ShortConv state
 * (float [(l_cache - 1)][n_embd], ring linearized) or the fp16 K rows then V
 * rows (full layers: positions 0 .. n-1; sliding-window layers: the last
 * min(n, window) positions in order), and a trailing FNV-1a 64 checksum of
 * everything after the header.  Files are byte-identical to the reference's.
 * The fields only the engine knows come in lfm_attn_cache_model. */
typedef struct {
    uint64_t model_fingerprint; /* lfm2_compute_model_fingerprint (tools/lfm2_sys_cache.c:394-422) */
    uint32_t n_model_layers;    /* ShortConv + attention layers (cfg.n_layers)      */
    uint32_t n_embd;            /* cfg.n_embd                                       */
    uint32_t n_head_q;          /* cfg.n_head_q (a header field)                    */
    uint32_t shortconv_l_cache; /* cfg.shortconv_l_cache                            */
    const int32_t *ctx_layer;   /* [n_model_layers]: this context's layer index of an
                                   attention layer, -1 for a ShortConv layer         */
} lfm_attn_cache_model;

/* Write a prompt cache of the first n_tokens positions
 * (lfm2_prompt_cache_save_ex, tools/lfm2_sys_cache.c:504-627): the
 * context's KV rows come from the device; conv_states[l] (host, ShortConv
 * layers) are linearized from their ring with conv_ring_heads (NULL: already
 * linear).  Written to "<path>.tmp.<pid>" and renamed over path.
 * LFM_ATTN_E_IO when the file cannot be written. */
int lfm_attn_ctx_cache_save(lfm_attn_ctx *ctx, const char *path, const lfm_attn_cache_model *model,
                            const uint32_t *tokens, uint32_t n_tokens, float *const *conv_states,
                            const uint32_t *conv_ring_heads);
/* Restore a prompt cache whose tokens are an exact prefix of prompt_tokens
 * (lfm2_prompt_cache_try_load_prefix_ex, tools/lfm2_sys_cache.c:650-797):
 * on success *matched_pos = the file's token count, the KV rows are in the
 * context's device caches, and conv_states[l] (when non-NULL) hold the
 * ShortConv states with out_conv_heads[l] = 0.  A file that does not apply
 * (missing, other model, longer than the prompt or max_seq, prefix mismatch,
 * truncated, bad checksum) returns LFM_ATTN_OK with *matched_pos = 0, as the
 * reference returns false; unlike the reference, the whole file is verified
 * before any cache or state is written, so a rejected file leaves them
 * untouched. */
int lfm_attn_ctx_cache_load_prefix(lfm_attn_ctx *ctx, const char *path,
                                   const lfm_attn_cache_model *model, const uint32_t *prompt_tokens,
                                   uint32_t n_prompt, float *const *conv_states,
                                   uint32_t *out_conv_heads, uint32_t *matched_pos);

/* ---- checkpoint SWA ring slab ------------------------------------------------
 * LFM2Checkpoint keeps, beside the ShortConv states and the position, a slab
 * of every sliding-window layer's whole ring: K [swa_cap][kv_dim] then V,
 * layer after layer in order (lfm2_checkpoint_save_ex / restore_ex,
 * tools/lfm2_moe_checkpoint.c:472-560; the slab is sized at :399-440 with
 * swa_cap = window + 8, which is what the engines use).  Here the rings are
 * the context's (swa_cap of the geometry).  The slab may be host or device
 * memory: a device slab makes a rollback an HBM-to-HBM copy.  Full-attention
 * layers need no snapshot: rewinding the position is enough. */
int lfm_attn_ctx_swa_slab_bytes(const lfm_attn_ctx *ctx, size_t *bytes);
int lfm_attn_ctx_swa_slab_save(lfm_attn_ctx *ctx, void *slab);
int lfm_attn_ctx_swa_slab_restore(lfm_attn_ctx *ctx, const void *slab);

/* Device address of a layer's caches (for callers that drive lfm_hip_* directly). */
int lfm_attn_ctx_kv_device(lfm_attn_ctx *ctx, uint32_t layer, uint16_t **k_dev, uint16_t **v_dev,
                           uint32_t *n_slots);

/* ---- achievable-peak probes (measurement only) --------------------------------
 * No counterpart in the reference: they measure this device's achievable
 * denominators for the roofline figures.  Asynchronous on `stream`.
 * lfm_hip_probe_read streams n_bytes (>= 16, 16-byte aligned) of device memory
 * with n_wg workgroups of 256 threads; sink receives n_wg words.
 * lfm_hip_probe_mfma runs n_wg workgroups of 4 waves, each wave `iters`
 * rounds of 8 independent 16x16x32 fp16 MFMAs (16,384 FLOPs each); out
 * receives n_wg * 256 floats. */
int lfm_hip_probe_read(const void *src, uint64_t n_bytes, uint32_t *sink, uint32_t n_wg,
                       lfm_attn_stream_t stream);
int lfm_hip_probe_mfma(float *out, uint32_t n_wg, uint32_t iters, lfm_attn_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LFM_ATTN_H */
