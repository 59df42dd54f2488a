/*
 * oracle/cpu_attn.h -- TEST INFRASTRUCTURE ONLY.
 *
 * A scalar C11 restatement of the reference CPU attention path
 * (avisheksharmacoder/laii), used as the parity checker for the HIP kernels
 * and as the "port" CPU baseline.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product library never does.
 *
 * Each function names the reference code it follows (file:line).  Where the
 * reference has several ISA variants of one algorithm (AVX2 / NEON / scalar)
 * the oracle follows the scalar variant's arithmetic; the variants differ only
 * in fp32 summation order.
 */
#ifndef LFM_ORACLE_CPU_ATTN_H
#define LFM_ORACLE_CPU_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- A8: IEEE binary16 <-> binary32 ------------------------------------ */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f); /* round-to-nearest-even, F16C semantics */
void     orc_f32_to_f16_n(const float *src, uint16_t *dst, size_t n);
void     orc_f16_to_f32_n(const uint16_t *src, float *dst, size_t n);

/* ---- A4/A5: RoPE tables ------------------------------------------------- */
void orc_rope_lut_lfm2(float *cos_lut, float *sin_lut, uint32_t max_seq,
                       uint32_t head_dim, float freq_base);
void orc_rope_lut_lfm3(float *cos_lut, float *sin_lut, uint32_t max_seq,
                       uint32_t head_dim, uint32_t rope_dim, float freq_base,
                       const float *rope_freqs, uint32_t n_rope_freqs);

/* ---- A4/A5: per-head RMSNorm + NeoX RoPE (+ RNE fp16 store) ------------- */
void orc_qk_norm_rope(float *vec, uint16_t *dst_f16, uint32_t n_heads,
                      uint32_t head_dim, const float *norm_w, float eps,
                      const float *cos_row, const float *sin_row);

/* ---- A4, production LFM2 stacks: float-angle table + lfm2_rmsnorm order - */
void orc_rope_table_lfm2(float *cos_tab, float *sin_tab, uint32_t max_seq,
                         uint32_t head_dim, float freq_base);
void orc_qk_norm_rope_table(float *vec, uint16_t *dst_f16, uint32_t n_heads,
                            uint32_t head_dim, const float *norm_w, float eps,
                            const float *cos_row, const float *sin_row);

/* ---- A1: LFM2 d=64 single-pass online softmax GQA ---------------------- */
void orc_online_gqa_f16(const float *q, const uint16_t *k_cache_f16,
                        const uint16_t *v_cache_f16, float *xb_out,
                        uint32_t n_head_q, uint32_t kv_mul, uint32_t kv_dim,
                        uint32_t pos, float scale);

/* ---- A2: per-head GQA task (FP16 online branch / FP32 two-pass) -------- */
void orc_gqa_heads(const float *q, const float *k_cache, const float *v_cache,
                   const uint16_t *k_cache_f16, const uint16_t *v_cache_f16,
                   float *xb, uint32_t n_head_q, uint32_t kv_mul,
                   uint32_t head_dim, uint32_t kv_dim, uint32_t pos, float scale);

/* ---- A3: LFM3 row plan + online GQA with SWA ring and output gate ------- */
void     orc_lfm3_plan(uint32_t abs_pos, uint32_t window_len, uint32_t swa_cap,
                       uint32_t out5[5]);
uint32_t orc_lfm3_slots(uint32_t abs_pos, uint32_t window_len, uint32_t swa_cap,
                        uint32_t *slots_out);
void orc_lfm3_online_gqa_f16(const float *q_batch, const float *gate_sig,
                             const uint16_t *k_cache_f16, const uint16_t *v_cache_f16,
                             float *xb_out, uint32_t B, uint32_t pos_0,
                             uint32_t window_len, uint32_t swa_cap,
                             uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim);

/* ---- A6: Gen-1 FP32 step (norm, per-call RoPE, FP32 append, two-pass) --- */
void orc_gen1_gqa_attend(float *attn_out, float *q, float *k, const float *v,
                         const float *q_norm, const float *k_norm,
                         float *k_cache, float *v_cache, uint32_t pos,
                         uint32_t n_heads_q, uint32_t n_heads_kv, uint32_t head_dim,
                         float eps, float theta);

/* ---- A7: causal batch (prefill / speculative verify) over FP16 KV ------- */
void orc_causal_rows_f16(const float *q_rows, const uint16_t *k_cache_f16,
                         const uint16_t *v_cache_f16, float *out_rows,
                         uint32_t n_rows, uint32_t pos_0, uint32_t n_head_q,
                         uint32_t n_head_kv, uint32_t head_dim);

/* ---- Next row: attention-sink eviction with RoPE counter-rotation ------- */
/* Host caches: k_caches[l] / v_caches[l] are [rows][n_head_kv[l] * head_dim]
 * fp16 bits (NULL or n_head_kv[l] == 0 = skipped layer); the LUTs are the
 * engine tables ([rows][head_dim / 2]).  Both return the new position.  The
 * rotation follows the AVX2 kernels (the default x86 build): lo' =
 * fma(lo, c, hi*s), hi' = fma(hi, c, -(lo*s)), RNE fp16. */
uint32_t orc_kv_shift_sinks_lfm2(uint16_t **k_caches, uint16_t **v_caches, uint32_t n_layers,
                                 const uint32_t *n_head_kv, uint32_t head_dim,
                                 const float *cos_lut, const float *sin_lut, uint32_t pos,
                                 uint32_t n_sink, uint32_t n_discard);
uint32_t orc_kv_shift_sinks_lfm3(uint16_t **k_caches, uint16_t **v_caches, uint32_t n_layers,
                                 const uint32_t *n_head_kv, const uint8_t *layer_kind,
                                 uint32_t head_dim, const float *cos_full, const float *sin_full,
                                 uint32_t full_rows, const float *cos_swa, const float *sin_swa,
                                 uint32_t swa_rows, uint32_t sliding_window, uint32_t swa_cap,
                                 uint32_t pos, uint32_t n_sink, uint32_t n_discard);

/* ---- Multi-threaded drivers (CPU baseline "port") ---------------------- */
/* Batched decode over n_seq independent caches; work items are
 * (sequence, 4-head group) pairs spread over n_threads pthreads. */
void orc_decode_batch_mt(const float *q, const uint16_t *const *k_seq,
                         const uint16_t *const *v_seq, const uint32_t *pos,
                         float *out, uint32_t n_seq, uint32_t n_head_q,
                         uint32_t n_head_kv, uint32_t head_dim, uint32_t n_threads);

/* ---- next-row projections: Q8_K activations, Q4_K x Q8_K matmul -------
 * Blocks are the reference's packed GGUF layouts:
 *   block_q4_K (144 B): fp16 d, fp16 dmin, scales[12] (6-bit scale/min pairs
 *                       of 8 sub-blocks), qs[128] (256 4-bit weights)
 *   block_q8_K (292 B): float d, int8 qs[256], int16 bsums[16]
 * (tools/lfm2_cpuid_quants.c:76-127). */
#define ORC_Q4K_BYTES 144u
#define ORC_Q8K_BYTES 292u

/* Q8_K of n_rows rows of n_cols floats (n_cols % 256 == 0), the AVX2
 * arithmetic the engine runs: d = max|x| / 127, q = round-half-even(x *
 * (127 / max|x|)), bsums of the unsaturated values
 * (lfm2_quantize_row_q8_K_avx2_cpuid, tools/lfm2_cpuid_quants.c:585-635;
 * per row as lfm2_quantize_batch_q8_K_avx2, tools/lfm2_prefill_batch.c:93-105). */
void orc_quantize_q8_K(const float *x, void *y, uint32_t n_rows, uint32_t n_cols);

/* One Q4_K row . Q8_K vector, in the order of lfm2_vec_dot_q4_K_q8_K_avx2
 * (include/lfm2_simd_avx2.h:364-412): exact integer sums per super-block,
 * then sumf += (d*d8)*dot - (dmin*d8)*mins, super-blocks in order. */
float orc_dot_q4_K_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols);

/* out[t][r] = row r of W . token t of x_q8 (lfm2_matmul_1x4_prequant_mt,
 * tools/lfm2_decode_1x4.c:795-813, B = 1; the Q4_K branch of
 * lfm2_matmul_batch_avx2_mt after its quantize step,
 * tools/lfm2_prefill_batch.c:479-510, 598-634). */
void orc_matmul_q4_K(float *out, const void *w, uint32_t n_rows, uint32_t n_cols,
                     const void *x_q8, uint32_t n_tokens);

/* block_q6_K (210 B): ql[128], qh[64], int8 scales[16], fp16 d.  One row .
 * Q8_K vector in the order of lfm2_vec_dot_q6_K_q8_K_avx2
 * (include/lfm2_simd_avx2.h:551-634): exact sum(sc*u*q8) and sum(sc*bsum)
 * per super-block, then sumf += (d*d8) * (float)(sum - 32*offset). */
#define ORC_Q6K_BYTES 210u
#define ORC_Q5K_BYTES 176u
#define ORC_IQ4XS_BYTES 136u
#define ORC_Q4_0_BYTES 18u /* per 32 weights */
#define ORC_Q8_0_BYTES 34u
float orc_dot_q4_0_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols);
float orc_dot_q8_0_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols);
float orc_dot_q5_K_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols);
float orc_dot_iq4_xs_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols);
size_t orc_q_row_bytes(uint32_t type, uint32_t n_cols); /* GGML type id */
float orc_dot_q6_K_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols);

/* out[t][r] for a matrix of GGML type 12 (Q4_K) or 14 (Q6_K). */
/* type: GGML id 2 (Q4_0), 8 (Q8_0), 12 (Q4_K), 13 (Q5_K), 14 (Q6_K), 23 (IQ4_XS) */
void orc_matmul_q(float *out, const void *w, uint32_t type, uint32_t n_rows, uint32_t n_cols,
                  const void *x_q8, uint32_t n_tokens);

/* ---- KV persistence (cpu_cache.c): .lfmcache v1 and the checkpoint slab -- */
/* layer_kind: 0 ShortConv, 1 full attention, 2 sliding-window attention */
uint64_t orc_fnv1a(uint64_t h, const void *data, size_t len);
uint64_t orc_model_fingerprint(const char *arch, uint32_t n_layers, uint32_t n_embd, uint32_t n_vocab,
                               uint32_t n_head_q, uint32_t l_cache, const uint32_t *n_head_kv, int is_lfm3,
                               uint32_t head_dim, uint32_t sliding_window, const uint8_t *is_swa);
int orc_prompt_cache_save(const char *path, uint64_t fingerprint, uint32_t n_layers, const uint32_t *n_head_kv,
                          const uint8_t *layer_kind, uint32_t head_dim, uint32_t n_embd, uint32_t n_head_q,
                          uint32_t l_cache, uint32_t sliding_window, const uint32_t *tokens, uint32_t n_tokens,
                          float *const *conv, const uint32_t *conv_heads, uint16_t *const *k, uint16_t *const *v,
                          uint32_t swa_cap);
uint32_t orc_prompt_cache_load(const char *path, uint64_t fingerprint, uint32_t n_layers,
                               const uint32_t *n_head_kv, const uint8_t *layer_kind, uint32_t head_dim,
                               uint32_t n_embd, uint32_t n_head_q, uint32_t l_cache, uint32_t sliding_window,
                               const uint32_t *prompt, uint32_t n_prompt, uint32_t max_seq, float *const *conv,
                               uint32_t *conv_heads, uint16_t *const *k, uint16_t *const *v, uint32_t swa_cap);
size_t orc_checkpoint_swa_slab(uint16_t *slab, uint32_t n_layers, const uint32_t *n_head_kv,
                               const uint8_t *layer_kind, uint32_t head_dim, uint32_t swa_cap,
                               uint16_t *const *k, uint16_t *const *v, int restore);

#ifdef __cplusplus
}
#endif
#endif /* LFM_ORACLE_CPU_ATTN_H */
