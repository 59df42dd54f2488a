/*
 * kernels.h -- internal interface between the extern "C" shim (shim.hip) and
 * the kernel translation units.  Not part of the public ABI.
 */
#ifndef LFM_ATTN_KERNELS_H
#define LFM_ATTN_KERNELS_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lfm {

/* One batch of attention rows over fp16 (or fp32) KV caches.
 * Sequence s uses cache k_seq[s] (device array) when k_seq != nullptr, else
 * k_base + s * seq_stride elements.  Its first row is position pos0_dev[s]
 * (device array) when pos0_dev != nullptr, else pos0_host. */
struct AttnBatch {
    const float *q            = nullptr; /* [n_seq][n_rows][n_head_q][head_dim]     */
    const float *gate         = nullptr; /* [n_seq][n_rows][n_head_q] or null       */
    int gate_is_logit         = 0;
    const void *k_base        = nullptr;
    const void *v_base        = nullptr;
    const void *const *k_seq  = nullptr;
    const void *const *v_seq  = nullptr;
    uint64_t seq_stride       = 0;       /* elements between sequences (k_base form) */
    const uint32_t *pos0_dev  = nullptr;
    uint32_t pos0_host        = 0;
    float *out                = nullptr; /* [n_seq][n_rows][n_head_q][head_dim]     */
    uint32_t out_dims         = 0;       /* dims written per head (<= head_dim)     */
    uint32_t n_seq = 1, n_rows = 1, n_head_q = 0, n_head_kv = 0, head_dim = 0;
    uint32_t window = 0, cap = 0;
    float scale = 0.0f;
    /* Fused prologue (the step entry): q holds the raw query rows, and the
     * kernel applies QK-RMSNorm + RoPE to q and to the raw new-token rows
     * k_new / v_new ([n_seq][n_rows][n_head_kv][head_dim]), which it also
     * stores as RNE fp16 at their slots.  k_new == nullptr: q is final and
     * the caches already hold every attended row. */
    const float *k_new = nullptr, *v_new = nullptr;
    const float *q_norm_w = nullptr, *k_norm_w = nullptr; /* [head_dim] or null (no norm) */
    const float *cos_lut = nullptr, *sin_lut = nullptr;   /* [position][head_dim / 2]     */
    float eps = 0.0f;
    int prologue = 0; /* LFM_PROLOGUE_FAST / LFM_PROLOGUE_TABLE: RMSNorm sum order */
};

/* Device workspace owned by the shim (grown on demand). */
void *workspace(size_t bytes, hipStream_t stream, int *status);

/* Device memory handed to a launch for its split partials in place of the
 * library workspace (the allocation-free entry point). */
struct Scratch {
    void *ptr;
    size_t bytes;
};

/* Split-KV MFMA kernel for fp16 caches, head_dim 64 or 128, up to 64 query
 * columns (n_rows * kv_mul) per KV head.  Returns LFM_ATTN_E_UNSUPPORTED for
 * other shapes (the caller then uses the generic kernel).  Split partials go
 * to `sc` when non-null (LFM_ATTN_E_SCRATCH, nothing launched, when they do
 * not fit), else to the library workspace. */
int launch_splitkv(const AttnBatch &b, uint32_t keys_hint, hipStream_t stream, const Scratch *sc = nullptr);
bool splitkv_supports(const AttnBatch &b);

/* Launch-plan overrides (tests, tuning): plan 0 automatic, 'g' grid, 'b'
 * balanced, 'd' balanced with LDS-streamed segments, 'w' in-workgroup
 * merge; 0 = automatic for the counts. */
struct Tuning {
    char plan;
    uint32_t waves, chunk, min_tiles;
    uint32_t prefill_chain; /* query tiles per sliding-window prefill workgroup */
};
int set_tuning(const char *plan, uint32_t waves, uint32_t chunk, uint32_t min_tiles, uint32_t prefill_chain);
/* "grid", "balanced", "balanced-dma" or "wg" for a PlanChoice kind */
const char *plan_name(char kind);
Tuning current_tuning();

/* The split-KV launch a batch takes on a device of `cus` compute units
 * (host only; of b it reads the shape, window and rows): kind 'w' (one workgroup per sequence and KV head, in-workgroup
 * merge), 'g' (fixed key chunks + merge kernel) or 'b' (tile shares + merge
 * kernel); waves per workgroup; grid key splits and chunk. */
struct PlanChoice {
    char kind;
    uint32_t waves, n_splits, chunk;
};
PlanChoice choose_plan(const AttnBatch &b, uint32_t keys_hint, bool positions_on_device, bool fuse, uint32_t cus,
                       const Tuning &t);

/* Generic one-wave-per-head kernel (any head_dim % 8 == 0, <= 256), fp16 or
 * fp32 caches; follows the reference's per-key recurrence. */
int launch_generic(const AttnBatch &b, bool kv_f32, hipStream_t stream);

/* Causal MFMA prefill (fp16 Q/K/V, fp32 out). */
bool prefill_supports(uint32_t head_dim, uint32_t kv_mul);
int launch_prefill(const float *q, const uint16_t *k, const uint16_t *v, float *out,
                   uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint64_t kv_seq_stride,
                   uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim, float scale,
                   hipStream_t stream);

/* Causal MFMA prefill for head_dim 128 with an optional sliding window and
 * output gate; K/V row r of a sequence's buffer holds position kv_pos0 + r. */
/* The launch shape of a head_dim-128/64 prefill (host only): query
 * positions per tile, tiles per workgroup, the short tiles at the sequence
 * start dispatched first, workgroups. */
struct PrefillExtPlan {
    uint32_t tq, chain, n_light, n_wg;
};
PrefillExtPlan prefill_ext_plan(uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint32_t window, uint32_t n_head_q,
                                uint32_t n_head_kv);
bool prefill_ext_supports(uint32_t head_dim, uint32_t kv_mul);
int launch_prefill_ext(const float *q, const uint16_t *k, const uint16_t *v, const float *gate, int gate_is_logit,
                       float *out, uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint32_t kv_pos0,
                       uint64_t kv_seq_stride, uint32_t window, uint32_t n_head_q, uint32_t n_head_kv,
                       uint32_t head_dim, float scale, hipStream_t stream);

/* Prologue kernels. */
int launch_qk_norm_rope(float *vec, uint16_t *dst_f16, uint32_t n_heads, uint32_t head_dim,
                        const float *norm_w, float eps, const float *cos_lut,
                        const float *sin_lut, uint32_t pos, int prologue, hipStream_t stream);
int launch_store_f16(uint16_t *dst, const float *src, uint32_t n, hipStream_t stream);
int launch_qkv_prologue(float *q, const float *k, const float *v, uint16_t *const *k_seq,
                        uint16_t *const *v_seq, const uint32_t *pos_0, uint32_t n_seq,
                        uint32_t n_rows, uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                        const float *q_norm_w, const float *k_norm_w, float eps,
                        const float *cos_lut, const float *sin_lut, uint32_t window_len,
                        uint32_t cap, int prologue, hipStream_t stream);

/* Gen-1 prologue (FP32 caches): Q normalised and rotated in place, K to
 * k_cache row pos, V copied to v_cache row pos. */
int launch_gen1_prologue(float *q, const float *k, const float *v, float *k_cache, float *v_cache,
                         const float *q_norm_w, const float *k_norm_w, float eps, const float *cos_row,
                         const float *sin_row, uint32_t pos, uint32_t n_head_q, uint32_t n_head_kv,
                         uint32_t head_dim, hipStream_t stream);

/* Projections beside the attention path (quant_matmul.hip).  y/x_q8:
 * packed block_q8_K rows; w: packed block_q4_K rows; n_cols % 256 == 0. */
int launch_quantize_q8_K(const float *x, void *y, uint32_t n_rows, uint32_t n_cols, hipStream_t stream);
/* Up to 4 matrices (GGML type 12 Q4_K or 14 Q6_K, rows[m] each) over the
 * same Q8_K tokens: outs[m][t][r]. */
int launch_matmul_q(uint32_t n_mats, float *const *outs, const void *const *ws, const uint32_t *types,
                    const uint32_t *rows, uint32_t n_cols, const void *x_q8, uint32_t n_tokens, hipStream_t stream);

/* Attention-sink eviction (kv_shift.hip).  launch_kv_shift moves rows
 * [n_sink + n_discard, n_sink + n_discard + n_keep) down to n_sink and
 * counter-rotates the keys; launch_kv_swa_repack re-slots an SWA ring
 * window through the staging rows stage_k / stage_v ([n_valid][kv_dim]). */
int launch_kv_shift(uint16_t *k, uint16_t *v, uint32_t kv_dim, uint32_t head_dim, uint32_t n_sink,
                    uint32_t n_keep, uint32_t n_discard, const float *cos_row, const float *sin_row,
                    hipStream_t stream);
int launch_kv_swa_repack(uint16_t *k, uint16_t *v, uint32_t kv_dim, uint32_t head_dim, uint32_t cap,
                         uint32_t t_start, uint32_t n_valid, uint32_t n_sink, uint32_t n_discard,
                         const float *cos_row, const float *sin_row, uint16_t *stage_k,
                         uint16_t *stage_v, hipStream_t stream);

/* Events recorded around the main attention kernel (null when off). */
void profile_events(hipEvent_t *before, hipEvent_t *after);

/* Record a HIP error for lfm_attn_last_error and map it to a status. */
int hip_status(hipError_t e);

/* Record the plan of this thread's last attention launch (a string literal)
 * for lfm_attn_last_plan. */
void note_plan(const char *name);

/* FNV-1a 64 of a device buffer (fnv_hash.hip). */
size_t fnv1a64_workspace_bytes(uint64_t len);
int launch_fnv1a64(const void *data, uint64_t len, uint64_t h_in, void *ws, hipStream_t stream);
uint64_t fnv1a64_finish(uint64_t h_in, uint64_t len, uint64_t acc);

/* Achievable-peak probes (peak_probe.hip). */
int launch_probe_read(const void *src, uint64_t n_bytes, uint32_t *sink, uint32_t n_wg, hipStream_t stream);
int launch_probe_mfma(float *out, uint32_t n_wg, uint32_t iters, hipStream_t stream);

} // namespace lfm

#endif
