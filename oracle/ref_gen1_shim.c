/*
 * oracle/ref_gen1_shim.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Exposes the reference's Gen-1 FP32 attention step (src/lfm_forward.c) as
 * plain C functions.  The reference's src/arena.c, lfm_simd.c, lfm_fused.c,
 * lfm_threadpool.c and lfm_forward.c are compiled where they lie under
 * /root/reference, one object each as its own Makefile does (nothing is
 * copied), and linked with this file, so tests can pin the oracle's Gen-1
 * restatement and the GPU path against the real lfm_gqa_step and
 * lfm_rope_neox.  Built by oracle/Makefile into oracle/_ref/libref_gen1.so,
 * only where /root/reference exists; the library travels with the tree.
 */
#define _GNU_SOURCE 1
#include <string.h>

#include "arena.h"
#include "lfm_forward.h"
#include "lfm_simd.h"

/* lfm_rope_neox(vec, head_dim, pos, theta) in place (src/lfm_forward.c:97-111). */
void ref_gen1_rope_neox(float *vec, uint32_t head_dim, uint32_t pos, float theta) {
    lfm_rope_neox(vec, head_dim, pos, theta);
}

/* lfm_vec_rmsnorm_f32(out, x, weight, n, eps) (src/lfm_simd.c:125-174). */
void ref_gen1_rmsnorm(float *out, const float *x, const float *weight, uint32_t n, float eps) {
    lfm_vec_rmsnorm_f32(out, x, weight, n, eps);
}

/* lfm_gqa_step with F32 weights: x_norm [D]; wq [nq*hd][D], wk, wv
 * [nkv*hd][D], wo [D][D]; caches [max_seq][nkv*hd] (row pos is appended);
 * out [D].  Returns 0, or -1 when the scratch arena cannot be set up. */
int ref_gen1_gqa_step(float *out, const float *x_norm, const float *wq, const float *wk, const float *wv,
                      const float *wo, const float *q_norm, const float *k_norm, float *k_cache, float *v_cache,
                      uint32_t pos, uint32_t max_seq, uint32_t D, uint32_t nq, uint32_t nkv, uint32_t hd,
                      float eps, float theta) {
    LFMConfig cfg;
    memset(&cfg, 0, sizeof cfg);
    cfg.hidden_dim  = D;
    cfg.n_heads_q   = nq;
    cfg.n_heads_kv  = nkv;
    cfg.head_dim    = hd;
    cfg.max_seq_len = max_seq;
    cfg.norm_eps    = eps;
    cfg.rope_theta  = theta;
    LFMLayerWeights lw;
    memset(&lw, 0, sizeof lw);
    lw.q_proj = wq;
    lw.q_proj_type = GGML_TYPE_F32;
    lw.k_proj = wk;
    lw.k_proj_type = GGML_TYPE_F32;
    lw.v_proj = wv;
    lw.v_proj_type = GGML_TYPE_F32;
    lw.q_norm = q_norm;
    lw.k_norm = k_norm;
    lw.attn_out_proj = wo;
    lw.attn_out_proj_type = GGML_TYPE_F32;
    LFMKVCache kv = {k_cache, v_cache};
    MemoryArena scratch;
    const size_t need = ((size_t)(nq + 3u * nkv + nq) * hd + (size_t)pos + 1u) * sizeof(float) + 64u * 1024u;
    if (!arena_init(&scratch, need)) return -1;
    lfm_gqa_step(out, x_norm, &lw, &kv, pos, &cfg, &scratch);
    arena_free(&scratch);
    return 0;
}
