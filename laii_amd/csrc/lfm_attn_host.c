/*
 * lfm_attn_host.c -- C11 host side of the attention path: the RoPE tables.
 *
 * The tables are built on the host in double precision exactly as the
 * reference builds them, so a table uploaded to HBM holds the same float bits
 * the reference's CPU kernels read:
 *   lfm2_rope_lut_init  tools/lfm2_kernels_fast.c:370-388
 *   lfm3_rope_lut_init  tools/lfm3_engine.c:403-450
 * The production LFM2 stacks (lfm2_forward.c, lfm2_prefill_batch.c) keep a
 * second table whose angles are float products, built at state init
 * (tools/lfm2_forward.c:572-581, tools/lfm2_prefill_batch.c:727-736):
 * lfm_attn_rope_table_lfm2 repeats those libm calls.
 * Layout [pos][head_dim/2], entry i rotating the pair (i, i + head_dim/2).
 * The Gen-1 engine has no table: lfm_rope_neox (src/lfm_forward.c:97-111)
 * recomputes one position's angles in float on every call, which
 * lfm_attn_rope_row_gen1 repeats with the same libm calls.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

#include "lfm_attn.h"

int lfm_attn_rope_lut_lfm2(float *cos_lut, float *sin_lut, uint32_t max_seq, uint32_t head_dim,
                           float freq_base) {
    if (!cos_lut || !sin_lut || head_dim == 0u || (head_dim & 1u)) return LFM_ATTN_E_INVALID;
    const uint32_t half = head_dim / 2u;
    for (uint32_t i = 0; i < half; ++i) {
        const double freq = pow((double)freq_base, -((double)(2u * i) / (double)head_dim));
        for (uint32_t p = 0; p < max_seq; ++p) {
            const double angle = (double)p * freq;
            cos_lut[(size_t)p * half + i] = (float)cos(angle);
            sin_lut[(size_t)p * half + i] = (float)sin(angle);
        }
    }
    return LFM_ATTN_OK;
}

int lfm_attn_rope_table_lfm2(float *cos_tab, float *sin_tab, uint32_t max_seq, uint32_t head_dim,
                             float freq_base) {
    if (!cos_tab || !sin_tab || head_dim == 0u || (head_dim & 1u)) return LFM_ATTN_E_INVALID;
    const uint32_t half = head_dim / 2u;
    const float base    = freq_base > 0.0f ? freq_base : 10000.0f;
    for (uint32_t i = 0; i < half; ++i) {
        const float freq = powf(base, -((float)(2u * i) / (float)head_dim));
        for (uint32_t p = 0; p < max_seq; ++p) {
            const float phi = (float)p * freq;
            cos_tab[(size_t)p * half + i] = cosf(phi);
            sin_tab[(size_t)p * half + i] = sinf(phi);
        }
    }
    return LFM_ATTN_OK;
}

int lfm_attn_rope_lut_lfm3(float *cos_lut, float *sin_lut, uint32_t max_seq, uint32_t head_dim,
                           uint32_t rope_dim, float freq_base, const float *rope_freqs,
                           uint32_t n_rope_freqs) {
    if (!cos_lut || !sin_lut || head_dim == 0u || (head_dim & 1u)) return LFM_ATTN_E_INVALID;
    const uint32_t half     = head_dim / 2u;
    const uint32_t rot_half = (rope_dim > 0u && rope_dim <= head_dim) ? rope_dim / 2u : half;
    for (uint32_t i = 0; i < half; ++i) {
        double freq = 0.0;
        if (i < rot_half) {
            freq = pow((double)freq_base, -((double)(2u * i) / (double)head_dim));
            if (rope_freqs && i < n_rope_freqs) {
                const double factor = (double)rope_freqs[i];
                /* a huge or non-positive factor switches the pair off */
                freq = (factor >= 1e10 || factor <= 0.0) ? 0.0 : freq / factor;
            }
        }
        for (uint32_t p = 0; p < max_seq; ++p) {
            float c = 1.0f, s = 0.0f;
            if (freq != 0.0) {
                const double angle = (double)p * freq;
                c = (float)cos(angle);
                s = (float)sin(angle);
            }
            cos_lut[(size_t)p * half + i] = c;
            sin_lut[(size_t)p * half + i] = s;
        }
    }
    return LFM_ATTN_OK;
}

int lfm_attn_rope_row_gen1(float *cos_row, float *sin_row, uint32_t head_dim, uint32_t pos, float theta) {
    if (!cos_row || !sin_row || head_dim == 0u || (head_dim & 1u)) return LFM_ATTN_E_INVALID;
    const uint32_t half = head_dim / 2u;
    for (uint32_t i = 0; i < half; ++i) {
        const float freq = 1.0f / powf(theta, (float)(2u * i) / (float)head_dim);
        const float phi  = (float)pos * freq;
        cos_row[i]       = cosf(phi);
        sin_row[i]       = sinf(phi);
    }
    return LFM_ATTN_OK;
}
