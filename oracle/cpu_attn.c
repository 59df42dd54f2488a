/*
 * oracle/cpu_attn.c -- TEST INFRASTRUCTURE ONLY (parity checker + "port" CPU
 * baseline).  Scalar C11 restatement of the reference attention path; see
 * cpu_attn.h.  Never linked into the product library.
 *
 * Pinning (what checks each function independently of this file):
 *   orc_f32_to_f16 / orc_f16_to_f32 : numpy float16 (IEEE RNE) over all 65536
 *                                     halves and random / tie / edge floats.
 *   orc_rope_lut_*                   : reference LUT builders compiled from
 *                                     source (oracle/_ref), closed form cos/sin,
 *                                     partial-RoPE identity pairs.
 *   orc_qk_norm_rope                 : reference AVX2/scalar kernels (oracle/_ref),
 *                                     numpy float64 closed form, norm invariant.
 *   orc_rope_table_lfm2,             : the reference's own table builders
 *   orc_qk_norm_rope_table             (lfm2_batch_state_init, lfm2_state_init) and
 *                                     prologues (lfm2_qk_norm_and_rope_table,
 *                                     lfm2_qk_norm_and_rope) compiled from source
 *                                     (oracle/_ref), bit-exact; float64 closed form.
 *   orc_online_gqa_f16, orc_gqa_heads, orc_lfm3_online_gqa_f16,
 *   orc_causal_rows_f16             : numpy float64 softmax(QK^T)V brute force,
 *                                     reference workers (oracle/_ref), golden
 *                                     vectors under tests/golden/.
 *   orc_lfm3_plan / orc_lfm3_slots   : brute-force window enumeration.
 *   orc_gen1_gqa_attend              : tests/fixtures_attention.bin (PyTorch).
 *   orc_kv_shift_sinks_lfm2 / _lfm3  : reference AVX2 shift kernels
 *                                     (oracle/_ref, bit-exact), rotation
 *                                     composition R(-d)R(p) = R(p-d) against
 *                                     keys roped at the new position, values
 *                                     moved unchanged, no-op cases.
 */
#define _GNU_SOURCE
#include "cpu_attn.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* A8: include/lfm2_simd_avx2.h:163-188 (IEEE half -> single).              */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp  = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x03FFu;
    uint32_t bits;
    if (exp == 0u) {
        if (mant == 0u) {
            bits = sign;
        } else {
            int e = -1;
            do { mant <<= 1; ++e; } while ((mant & 0x0400u) == 0u);
            mant &= 0x03FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31u) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + (127u - 15u)) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* A8: the F16C store used by every KV write in the reference
 * (_mm256_cvtps_ph(..., _MM_FROUND_TO_NEAREST_INT), tools/lfm2_kernels_fast.c:477-484,
 * 505; tools/lfm3_engine.c:518-519): IEEE round-to-nearest-even, overflow to
 * infinity, NaN stays NaN (quieted). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax   = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {
        if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x03FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    if (ax >= 0x38800000u) { /* |f| >= 2^-14: normal half or overflow */
        uint32_t h   = ((ax >> 23) - 112u) << 10 | ((ax >> 13) & 0x03FFu);
        uint32_t rem = ax & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
        if (h >= 0x7C00u) h = 0x7C00u;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to zero */
    /* subnormal half: value / 2^-24 = m * 2^(E-126) with E <= 112 */
    const uint32_t E     = ax >> 23;
    const uint32_t m     = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - E;
    uint32_t q           = m >> shift;
    const uint32_t rem   = m & ((1u << shift) - 1u);
    const uint32_t half  = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

void orc_f32_to_f16_n(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_n(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* A4: tools/lfm2_kernels_fast.c:370-388 -- double-precision angle, float
 * entries, layout [pos][head_dim/2]. */
void orc_rope_lut_lfm2(float *cos_lut, float *sin_lut, uint32_t max_seq,
                       uint32_t head_dim, float freq_base) {
    const uint32_t half = head_dim / 2u;
    for (uint32_t i = 0; i < half; ++i) {
        const double freq = pow((double)freq_base, -((double)(2u * i) / (double)head_dim));
        for (uint32_t p = 0; p < max_seq; ++p) {
            const double angle = (double)p * freq;
            cos_lut[(size_t)p * half + i] = (float)cos(angle);
            sin_lut[(size_t)p * half + i] = (float)sin(angle);
        }
    }
}

/* A5: tools/lfm3_engine.c:403-450 -- partial RoPE: pairs i >= rope_dim/2, and
 * pairs whose rope_freqs factor is >= 1e10 or <= 0, get the identity
 * rotation (cos 1, sin 0); other frequencies are divided by the factor. */
void orc_rope_lut_lfm3(float *cos_lut, float *sin_lut, uint32_t max_seq,
                       uint32_t head_dim, uint32_t rope_dim, float freq_base,
                       const float *rope_freqs, uint32_t n_rope_freqs) {
    const uint32_t half     = head_dim / 2u;
    const uint32_t rot_half = (rope_dim > 0u && rope_dim <= head_dim) ? (rope_dim / 2u) : half;
    for (uint32_t i = 0; i < half; ++i) {
        double freq = 0.0;
        if (i < rot_half) {
            freq = pow((double)freq_base, -((double)(2u * i) / (double)head_dim));
            if (rope_freqs != NULL && i < n_rope_freqs) {
                const double sf = (double)rope_freqs[i];
                if (sf >= 1e10 || sf <= 0.0) freq = 0.0;
                else freq /= sf;
            }
        }
        for (uint32_t p = 0; p < max_seq; ++p) {
            if (freq == 0.0) {
                cos_lut[(size_t)p * half + i] = 1.0f;
                sin_lut[(size_t)p * half + i] = 0.0f;
            } else {
                const double angle = (double)p * freq;
                cos_lut[(size_t)p * half + i] = (float)cos(angle);
                sin_lut[(size_t)p * half + i] = (float)sin(angle);
            }
        }
    }
}

/* A4/A5: tools/lfm2_kernels_fast.c:511-547 (scalar LFM2, double sum of
 * squares) generalised to any even head_dim as in tools/lfm3_engine.c:599-642:
 * x <- (x * irms) * w with irms = 1/sqrtf(mean(x^2) + eps); NeoX rotation of
 * pairs (i, i + head_dim/2); with dst_f16 the rotated head is stored as RNE
 * fp16 and vec is left untouched, otherwise vec is overwritten. */
/* Sum of squares of one head in the order of the reference's AVX2 kernels
 * (eight vector columns j, then a horizontal sum), which the engine runs:
 *   64  lfm2_qk_norm_rope_avx2, tools/lfm2_kernels_fast.c:443-449, hsum of
 *       include/lfm2_simd_avx2.h:286-293;
 *   128 lfm3_qk_norm_rope_128_avx2, tools/lfm3_engine.c:480-494.
 * Other head dims: the scalar kernels' double sum
 * (tools/lfm2_kernels_fast.c:527-529). */
static float sumsq_ref(const float *x, uint32_t head_dim) {
    float t[8];
    if (head_dim == 64u) {
        for (int j = 0; j < 8; ++j) {
            float ss0 = x[j] * x[j] + x[32 + j] * x[32 + j];
            float ss1 = x[8 + j] * x[8 + j] + x[40 + j] * x[40 + j];
            ss0 = fmaf(x[16 + j], x[16 + j], fmaf(x[48 + j], x[48 + j], ss0));
            ss1 = fmaf(x[24 + j], x[24 + j], fmaf(x[56 + j], x[56 + j], ss1));
            t[j] = ss0 + ss1;
        }
        return ((t[0] + t[4]) + (t[2] + t[6])) + ((t[1] + t[5]) + (t[3] + t[7]));
    }
    if (head_dim == 128u) {
        for (int j = 0; j < 8; ++j) {
            float ss0 = 0.0f, ss1 = 0.0f;
            for (int i = 0; i < 128; i += 16) {
                ss0 = fmaf(x[i + j], x[i + j], ss0);
                ss1 = fmaf(x[i + 8 + j], x[i + 8 + j], ss1);
            }
            t[j] = ss0 + ss1;
        }
        return ((t[0] + t[4]) + (t[1] + t[5])) + ((t[2] + t[6]) + (t[3] + t[7]));
    }
    double ss = 0.0;
    for (uint32_t i = 0; i < head_dim; ++i) ss += (double)x[i] * (double)x[i];
    return (float)ss;
}

void orc_qk_norm_rope(float *vec, uint16_t *dst_f16, uint32_t n_heads,
                      uint32_t head_dim, const float *norm_w, float eps,
                      const float *cos_row, const float *sin_row) {
    const uint32_t half = head_dim / 2u;
    float tmp[512];
    for (uint32_t h = 0; h < n_heads; ++h) {
        const float *hp = vec + (size_t)h * head_dim;
        for (uint32_t i = 0; i < head_dim; ++i) tmp[i] = hp[i];
        if (norm_w != NULL) {
            const float ss   = sumsq_ref(tmp, head_dim);
            const float irms = 1.0f / sqrtf(ss / (float)head_dim + eps);
            for (uint32_t i = 0; i < head_dim; ++i) tmp[i] = (tmp[i] * irms) * norm_w[i];
        }
        /* the AVX2 kernels (head_dim 64, 128) rotate with fmsub / fmadd,
         * the scalar kernels with separately rounded products */
        const int fused = head_dim == 64u || head_dim == 128u;
        for (uint32_t i = 0; i < half; ++i) {
            const float x0 = tmp[i], x1 = tmp[i + half];
            const float c = cos_row[i], s = sin_row[i];
            const float r0 = fused ? fmaf(x0, c, -(x1 * s)) : x0 * c - x1 * s;
            const float r1 = fused ? fmaf(x1, c, x0 * s) : x1 * c + x0 * s;
            if (dst_f16 != NULL) {
                dst_f16[(size_t)h * head_dim + i]        = orc_f32_to_f16(r0);
                dst_f16[(size_t)h * head_dim + i + half] = orc_f32_to_f16(r1);
            } else {
                vec[(size_t)h * head_dim + i]        = r0;
                vec[(size_t)h * head_dim + i + half] = r1;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* A4, the production LFM2 stacks (lfm2_forward.c, lfm2_prefill_batch.c):
 * float-angle table of lfm2_state_init / lfm2_batch_state_init
 * (tools/lfm2_forward.c:572-581, tools/lfm2_prefill_batch.c:727-736):
 * freq_i = powf(base, -((float)(2i) / (float)head_dim)), angle = (float)p *
 * freq_i in float, entries cosf / sinf of it; base <= 0 means 10000. */
void orc_rope_table_lfm2(float *cos_tab, float *sin_tab, uint32_t max_seq,
                         uint32_t head_dim, float freq_base) {
    const uint32_t half = head_dim / 2u;
    const float base = freq_base > 0.0f ? freq_base : 10000.0f;
    for (uint32_t i = 0; i < half; ++i) {
        const float freq = powf(base, -((float)(2u * i) / (float)head_dim));
        for (uint32_t p = 0; p < max_seq; ++p) {
            const float angle = (float)p * freq;
            cos_tab[(size_t)p * half + i] = cosf(angle);
            sin_tab[(size_t)p * half + i] = sinf(angle);
        }
    }
}

/* A4, the production LFM2 stacks: lfm2_qk_norm_and_rope_table
 * (tools/lfm2_prefill_batch.c:826-893) and lfm2_qk_norm_and_rope
 * (tools/lfm2_forward.c:775-830) of the AVX2 build.  Per head, lfm2_rmsnorm
 * (tools/lfm2_forward.c:669-706): eight fp32 accumulators, column j a fused
 * multiply-add chain over dims 8k + j of every full group of eight, the
 * columns then added in order 0..7 in double, dims past the last full group
 * added in double one at a time; irms = 1/sqrtf((float)(ss / dim) + eps);
 * x <- (x * irms) * w.  Rotation of pairs (i, i + half): pairs in full groups
 * of eight use fmsub / fmadd (lo' = fma(lo, c, -(hi*s)), hi' = fma(hi, c,
 * lo*s)), the rest separately rounded products.  Stores as orc_qk_norm_rope. */
void orc_qk_norm_rope_table(float *vec, uint16_t *dst_f16, uint32_t n_heads,
                            uint32_t head_dim, const float *norm_w, float eps,
                            const float *cos_row, const float *sin_row) {
    const uint32_t half = head_dim / 2u;
    const uint32_t full = head_dim & ~7u, full_half = half & ~7u;
    float tmp[512];
    for (uint32_t h = 0; h < n_heads; ++h) {
        const float *hp = vec + (size_t)h * head_dim;
        for (uint32_t i = 0; i < head_dim; ++i) tmp[i] = hp[i];
        if (norm_w != NULL) {
            float col[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (uint32_t d = 0; d < full; d += 8u)
                for (uint32_t j = 0; j < 8u; ++j) col[j] = fmaf(tmp[d + j], tmp[d + j], col[j]);
            double ss = 0.0;
            for (uint32_t j = 0; j < 8u; ++j) ss += (double)col[j];
            for (uint32_t d = full; d < head_dim; ++d) ss += (double)tmp[d] * (double)tmp[d];
            const float irms = 1.0f / sqrtf((float)(ss / (double)head_dim) + eps);
            for (uint32_t i = 0; i < head_dim; ++i) tmp[i] = (tmp[i] * irms) * norm_w[i];
        }
        for (uint32_t i = 0; i < half; ++i) {
            const float x0 = tmp[i], x1 = tmp[i + half];
            const float c = cos_row[i], s = sin_row[i];
            const int fused = i < full_half;
            const float r0 = fused ? fmaf(x0, c, -(x1 * s)) : x0 * c - x1 * s;
            const float r1 = fused ? fmaf(x1, c, x0 * s) : x1 * c + x0 * s;
            if (dst_f16 != NULL) {
                dst_f16[(size_t)h * head_dim + i]        = orc_f32_to_f16(r0);
                dst_f16[(size_t)h * head_dim + i + half] = orc_f32_to_f16(r1);
            } else {
                vec[(size_t)h * head_dim + i]        = r0;
                vec[(size_t)h * head_dim + i + half] = r1;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* One query head streamed over a contiguous run of cache rows with the
 * reference's single-pass recurrence (tools/lfm2_kernels_fast.c:845-866,
 * tools/lfm3_engine.c:1068-1089): a larger score rescales the running sums by
 * alpha = expf(m - s) (0 on the first key, m <= -1e29), a smaller one adds
 * beta = expf(s - m).  Updates vo[0..head_dim), *m, *l in place. */
static void orc_head_segment(const float *q_h, const uint16_t *k_ptr, const uint16_t *v_ptr,
                             size_t stride, uint32_t seg_len, uint32_t head_dim, float scale,
                             float *vo, float *m_p, float *l_p) {
    float m = *m_p, l = *l_p;
    for (uint32_t t = 0; t < seg_len; ++t) {
        float dot = 0.0f;
        for (uint32_t i = 0; i < head_dim; ++i) dot += q_h[i] * orc_f16_to_f32(k_ptr[i]);
        const float score = dot * scale;
        if (score > m) {
            const float alpha = (m <= -1e29f) ? 0.0f : expf(m - score);
            l = l * alpha + 1.0f;
            m = score;
            for (uint32_t i = 0; i < head_dim; ++i) vo[i] = vo[i] * alpha + orc_f16_to_f32(v_ptr[i]);
        } else {
            const float beta = expf(score - m);
            l += beta;
            for (uint32_t i = 0; i < head_dim; ++i) vo[i] += beta * orc_f16_to_f32(v_ptr[i]);
        }
        k_ptr += stride;
        v_ptr += stride;
    }
    *m_p = m;
    *l_p = l;
}

/* A1: tools/lfm2_kernels_fast.c:814-872 (scalar worker; the AVX2 worker
 * :700-810 is the same recurrence).  head_dim is 64; kv_h = h / kv_mul; the
 * output is vo * (1/l).  All ceil(n_head_q/4) work items are run in order. */
void orc_online_gqa_f16(const float *q, const uint16_t *k_cache_f16,
                        const uint16_t *v_cache_f16, float *xb_out,
                        uint32_t n_head_q, uint32_t kv_mul, uint32_t kv_dim,
                        uint32_t pos, float scale) {
    for (uint32_t h = 0; h < n_head_q; ++h) {
        const uint32_t kv_h = h / kv_mul;
        float vo[64] = {0.0f};
        float m = -1e30f, l = 0.0f;
        orc_head_segment(q + (size_t)h * 64u, k_cache_f16 + (size_t)kv_h * 64u,
                         v_cache_f16 + (size_t)kv_h * 64u, kv_dim, pos + 1u, 64u, scale,
                         vo, &m, &l);
        const float inv_l = 1.0f / l;
        for (uint32_t i = 0; i < 64u; ++i) xb_out[(size_t)h * 64u + i] = vo[i] * inv_l;
    }
}

/* A2: tools/lfm2_threadpool.c:764-931.  FP16 branch (:778-828): the shifted
 * recurrence (expf(-1e30 - s) == 0 on the first key), output vo * (l>0 ? 1/l : 0)
 * over n_vec*8 dims with n_vec = (head_dim <= 64) ? head_dim/8 : 8, i.e. only
 * the first 64 dims when head_dim > 64 (reference quirk, reproduced).
 * FP32 branch (:887-928, taken when the f16 caches are NULL): two-pass
 * softmax -- scores, max, expf, normalise by 1/sum, weighted V sum in t order. */
void orc_gqa_heads(const float *q, const float *k_cache, const float *v_cache,
                   const uint16_t *k_cache_f16, const uint16_t *v_cache_f16,
                   float *xb, uint32_t n_head_q, uint32_t kv_mul,
                   uint32_t head_dim, uint32_t kv_dim, uint32_t pos, float scale) {
    for (uint32_t h = 0; h < n_head_q; ++h) {
        const float *q_head = q + (size_t)h * head_dim;
        const uint32_t kv_h = h / kv_mul;
        float *out_head     = xb + (size_t)h * head_dim;
        if (k_cache_f16 != NULL && v_cache_f16 != NULL) {
            const uint32_t n_out = (head_dim <= 64u) ? head_dim : 64u;
            float vo[512] = {0.0f};
            float m = -1e30f, l = 0.0f;
            for (uint32_t t = 0; t <= pos; ++t) {
                const uint16_t *kt = k_cache_f16 + (size_t)t * kv_dim + (size_t)kv_h * head_dim;
                const uint16_t *vt = v_cache_f16 + (size_t)t * kv_dim + (size_t)kv_h * head_dim;
                float dot = 0.0f;
                for (uint32_t i = 0; i < head_dim; ++i) dot += q_head[i] * orc_f16_to_f32(kt[i]);
                const float s = dot * scale;
                if (s > m) {
                    const float sp = expf(m - s);
                    m = s;
                    l = l * sp + 1.0f;
                    for (uint32_t i = 0; i < n_out; ++i) vo[i] = vo[i] * sp + orc_f16_to_f32(vt[i]);
                } else {
                    const float w = expf(s - m);
                    l += w;
                    for (uint32_t i = 0; i < n_out; ++i) vo[i] += orc_f16_to_f32(vt[i]) * w;
                }
            }
            const float inv_l = (l > 0.0f) ? (1.0f / l) : 0.0f;
            for (uint32_t i = 0; i < n_out; ++i) out_head[i] = vo[i] * inv_l;
            continue;
        }
        float *scores = (float *)malloc(((size_t)pos + 1u) * sizeof(float));
        float max_score = -1e30f;
        for (uint32_t t = 0; t <= pos; ++t) {
            const float *k_t = k_cache + (size_t)t * kv_dim + (size_t)kv_h * head_dim;
            float dot = 0.0f;
            for (uint32_t i = 0; i < head_dim; ++i) dot += q_head[i] * k_t[i];
            scores[t] = dot * scale;
            if (scores[t] > max_score) max_score = scores[t];
        }
        float sum_exp = 0.0f;
        for (uint32_t t = 0; t <= pos; ++t) {
            scores[t] = expf(scores[t] - max_score);
            sum_exp += scores[t];
        }
        const float inv_sum = 1.0f / sum_exp;
        for (uint32_t t = 0; t <= pos; ++t) scores[t] *= inv_sum;
        for (uint32_t i = 0; i < head_dim; ++i) out_head[i] = 0.0f;
        for (uint32_t t = 0; t <= pos; ++t) {
            const float *v_t = v_cache + (size_t)t * kv_dim + (size_t)kv_h * head_dim;
            for (uint32_t i = 0; i < head_dim; ++i) out_head[i] += scores[t] * v_t[i];
        }
        free(scores);
    }
}

/* ------------------------------------------------------------------------ */
/* A3 row plan, literally tools/lfm3_engine.c:1073-1080 (== :862-873). */
void orc_lfm3_plan(uint32_t abs_pos, uint32_t window_len, uint32_t swa_cap, uint32_t out5[5]) {
    const uint32_t t_start = (window_len > 0u && abs_pos + 1u > window_len)
                           ? (abs_pos + 1u - window_len) : 0u;
    const uint32_t count     = abs_pos - t_start + 1u;
    const uint32_t seg1_slot = (window_len > 0u) ? (t_start % swa_cap) : t_start;
    const uint32_t seg1_len  = (window_len > 0u && seg1_slot + count > swa_cap)
                             ? (swa_cap - seg1_slot) : count;
    out5[0] = t_start;
    out5[1] = count;
    out5[2] = seg1_slot;
    out5[3] = seg1_len;
    out5[4] = count - seg1_len;
}

/* Slots in the order the reference workers visit them: seg1 from seg1_slot,
 * then seg2 from slot 0 (tools/lfm3_engine.c:1103-1114).  Returns count. */
uint32_t orc_lfm3_slots(uint32_t abs_pos, uint32_t window_len, uint32_t swa_cap,
                        uint32_t *slots_out) {
    uint32_t p[5];
    orc_lfm3_plan(abs_pos, window_len, swa_cap, p);
    uint32_t n = 0;
    for (uint32_t t = 0; t < p[3]; ++t) slots_out[n++] = p[2] + t;
    for (uint32_t t = 0; t < p[4]; ++t) slots_out[n++] = t;
    return n;
}

/* A3: tools/lfm3_engine.c:1116-1153 (scalar worker) + :1155-1204 (dispatch:
 * kv_mul = n_head_q / n_head_kv, scale = 1/sqrtf(head_dim)).  Row b is query
 * position pos_0 + b; output = vo * (l > 0 ? gate/l : 0) with gate = 1 when
 * gate_sig is NULL. */
void orc_lfm3_online_gqa_f16(const float *q_batch, const float *gate_sig,
                             const uint16_t *k_cache_f16, const uint16_t *v_cache_f16,
                             float *xb_out, uint32_t B, uint32_t pos_0,
                             uint32_t window_len, uint32_t swa_cap,
                             uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim) {
    const uint32_t kv_mul = (n_head_kv > 0u) ? (n_head_q / n_head_kv) : 1u;
    const size_t stride   = (size_t)n_head_kv * head_dim;
    const float scale     = 1.0f / sqrtf((float)head_dim);
    for (uint32_t b = 0; b < B; ++b) {
        uint32_t p[5];
        orc_lfm3_plan(pos_0 + b, window_len, swa_cap, p);
        const float *q_tok = q_batch + (size_t)b * n_head_q * head_dim;
        float *o_tok       = xb_out + (size_t)b * n_head_q * head_dim;
        const float *g_tok = gate_sig ? gate_sig + (size_t)b * n_head_q : NULL;
        for (uint32_t h = 0; h < n_head_q; ++h) {
            const size_t kv_off = (size_t)(h / kv_mul) * head_dim;
            float vo[512] = {0.0f};
            float m = -1e30f, l = 0.0f;
            orc_head_segment(q_tok + (size_t)h * head_dim,
                             k_cache_f16 + (size_t)p[2] * stride + kv_off,
                             v_cache_f16 + (size_t)p[2] * stride + kv_off,
                             stride, p[3], head_dim, scale, vo, &m, &l);
            if (p[4] > 0u) {
                orc_head_segment(q_tok + (size_t)h * head_dim, k_cache_f16 + kv_off,
                                 v_cache_f16 + kv_off, stride, p[4], head_dim, scale,
                                 vo, &m, &l);
            }
            const float gv    = g_tok ? g_tok[h] : 1.0f;
            const float inv_l = (l > 0.0f) ? (gv / l) : 0.0f;
            for (uint32_t i = 0; i < head_dim; ++i) o_tok[(size_t)h * head_dim + i] = vo[i] * inv_l;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Gen-1 AVX2 helpers in their exact summation order.
 * hsum256_ps (src/lfm_simd.c:51-58): columns k and k + 4 added, then the four
 * sums one after another. */
static float gen1_hsum8(const float *c) {
    const float b0 = c[0] + c[4], b1 = c[1] + c[5], b2 = c[2] + c[6], b3 = c[3] + c[7];
    return ((b0 + b1) + b2) + b3;
}

/* Sum of squares of lfm_vec_rmsnorm_f32 (src/lfm_simd.c:125-145): eight
 * columns j accumulate fma over dims 32b + j, +8, +16, +24 of each full
 * 32-block, then hsum256_ps, then the remaining dims one at a time. */
static float gen1_sumsq(const float *x, uint32_t n) {
    float col[8] = {0};
    uint32_t i = 0;
    for (; i + 32u <= n; i += 32u)
        for (uint32_t q = 0; q < 4u; ++q)
            for (uint32_t j = 0; j < 8u; ++j) col[j] = fmaf(x[i + 8u * q + j], x[i + 8u * q + j], col[j]);
    float s = gen1_hsum8(col);
    for (; i < n; ++i) s += x[i] * x[i];
    return s;
}

/* lfm_vec_dot_f32 (src/lfm_simd.c:61-83): four 8-column accumulators over the
 * dims 32b + j, +8, +16, +24, combined (acc0 + acc1) + (acc2 + acc3), hsum,
 * then the remaining dims one at a time. */
static float gen1_dot(const float *a, const float *b, uint32_t n) {
    float acc[4][8] = {{0}};
    uint32_t i = 0;
    for (; i + 32u <= n; i += 32u)
        for (uint32_t q = 0; q < 4u; ++q)
            for (uint32_t j = 0; j < 8u; ++j) acc[q][j] = fmaf(a[i + 8u * q + j], b[i + 8u * q + j], acc[q][j]);
    float t[8];
    for (uint32_t j = 0; j < 8u; ++j) t[j] = (acc[0][j] + acc[1][j]) + (acc[2][j] + acc[3][j]);
    float s = gen1_hsum8(t);
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}

/* A6: src/lfm_forward.c:181-244 after the projections.  RMSNorm per
 * src/lfm_simd.c:125-170 (the AVX2 sum of squares above, x * r * w), RoPE
 * per src/lfm_forward.c:97-111 (float powf/cosf/sinf per call, separately
 * rounded products), FP32 append at pos (:198-202), two-pass softmax
 * attention with lfm_vec_dot_f32 scores (:204-244). */
void orc_gen1_gqa_attend(float *attn_out, float *q, float *k, const float *v,
                         const float *q_norm, const float *k_norm,
                         float *k_cache, float *v_cache, uint32_t pos,
                         uint32_t n_heads_q, uint32_t n_heads_kv, uint32_t head_dim,
                         float eps, float theta) {
    const uint32_t half  = head_dim / 2u;
    const uint32_t group = n_heads_q / n_heads_kv;
    for (uint32_t pass = 0; pass < 2u; ++pass) {
        float *vec          = pass == 0u ? q : k;
        const float *w      = pass == 0u ? q_norm : k_norm;
        const uint32_t nh   = pass == 0u ? n_heads_q : n_heads_kv;
        for (uint32_t h = 0; h < nh; ++h) {
            float *x = vec + (size_t)h * head_dim;
            const float ss = gen1_sumsq(x, head_dim);
            const float r  = 1.0f / sqrtf((ss / (float)head_dim) + eps);
            for (uint32_t i = 0; i < head_dim; ++i) x[i] = w ? x[i] * r * w[i] : x[i] * r;
            for (uint32_t i = 0; i < half; ++i) {
                const float freq = 1.0f / powf(theta, (float)(2u * i) / (float)head_dim);
                const float phi  = (float)pos * freq;
                const float c = cosf(phi), s = sinf(phi);
                const float x0 = x[i], x1 = x[i + half];
                x[i]        = x0 * c - x1 * s;
                x[i + half] = x1 * c + x0 * s;
            }
        }
    }
    const size_t kv_dim = (size_t)n_heads_kv * head_dim;
    memcpy(k_cache + (size_t)pos * kv_dim, k, kv_dim * sizeof(float));
    memcpy(v_cache + (size_t)pos * kv_dim, v, kv_dim * sizeof(float));
    const float scale = 1.0f / sqrtf((float)head_dim);
    float *scores = (float *)malloc(((size_t)pos + 1u) * sizeof(float));
    for (uint32_t hq = 0; hq < n_heads_q; ++hq) {
        const uint32_t hkv = hq / group;
        const float *qh = q + (size_t)hq * head_dim;
        float *out_h = attn_out + (size_t)hq * head_dim;
        memset(out_h, 0, head_dim * sizeof(float));
        float max_score = -1e30f;
        for (uint32_t t = 0; t <= pos; ++t) {
            const float *kt = k_cache + (size_t)t * kv_dim + (size_t)hkv * head_dim;
            scores[t] = gen1_dot(qh, kt, head_dim) * scale;
            if (scores[t] > max_score) max_score = scores[t];
        }
        float sum_exp = 0.0f;
        for (uint32_t t = 0; t <= pos; ++t) {
            scores[t] = expf(scores[t] - max_score);
            sum_exp += scores[t];
        }
        const float inv_sum = 1.0f / sum_exp;
        for (uint32_t t = 0; t <= pos; ++t) scores[t] *= inv_sum;
        for (uint32_t t = 0; t <= pos; ++t) {
            const float *vt = v_cache + (size_t)t * kv_dim + (size_t)hkv * head_dim;
            for (uint32_t d = 0; d < head_dim; ++d) out_h[d] += scores[t] * vt[d];
        }
    }
    free(scores);
}

/* A7: tools/lfm2_prefill_batch.c:1029-1092 -- row r is position pos_0 + r and
 * attends [0, pos_0 + r] through the per-head task (FP16 branch), one row at
 * a time; the cache must already hold rows 0 .. pos_0 + n_rows - 1. */
void orc_causal_rows_f16(const float *q_rows, const uint16_t *k_cache_f16,
                         const uint16_t *v_cache_f16, float *out_rows,
                         uint32_t n_rows, uint32_t pos_0, uint32_t n_head_q,
                         uint32_t n_head_kv, uint32_t head_dim) {
    const uint32_t kv_dim = n_head_kv * head_dim;
    const float scale     = 1.0f / sqrtf((float)head_dim);
    for (uint32_t r = 0; r < n_rows; ++r) {
        orc_gqa_heads(q_rows + (size_t)r * n_head_q * head_dim, NULL, NULL, k_cache_f16,
                      v_cache_f16, out_rows + (size_t)r * n_head_q * head_dim, n_head_q,
                      n_head_q / n_head_kv, head_dim, kv_dim, pos_0 + r, scale);
    }
}

/* ------------------------------------------------------------------------ */
/* Threaded batched decode: the reference's work item (4 query heads,
 * tools/lfm2_kernels_fast.c:706-710) claimed dynamically like
 * lfm2_threadpool_claim_chunk (tools/lfm2_threadpool.c:506-520), but over all
 * (sequence, head group) pairs of the batch. */
typedef struct {
    const float *q;
    const uint16_t *const *k_seq;
    const uint16_t *const *v_seq;
    const uint32_t *pos;
    float *out;
    uint32_t n_seq, n_head_q, n_head_kv, head_dim, n_groups;
    atomic_uint next;
} orc_batch_job;

static void *orc_batch_worker(void *arg) {
    orc_batch_job *j = (orc_batch_job *)arg;
    const uint32_t kv_mul = j->n_head_q / j->n_head_kv;
    const size_t stride   = (size_t)j->n_head_kv * j->head_dim;
    const float scale     = 1.0f / sqrtf((float)j->head_dim);
    float vo[512];
    for (;;) {
        const uint32_t item = atomic_fetch_add_explicit(&j->next, 1u, memory_order_relaxed);
        if (item >= j->n_seq * j->n_groups) break;
        const uint32_t s = item / j->n_groups, g = item % j->n_groups;
        const uint32_t h_end = (g * 4u + 4u < j->n_head_q) ? g * 4u + 4u : j->n_head_q;
        for (uint32_t h = g * 4u; h < h_end; ++h) {
            const size_t kv_off = (size_t)(h / kv_mul) * j->head_dim;
            const size_t qo     = ((size_t)s * j->n_head_q + h) * j->head_dim;
            float m = -1e30f, l = 0.0f;
            memset(vo, 0, j->head_dim * sizeof(float));
            orc_head_segment(j->q + qo, j->k_seq[s] + kv_off, j->v_seq[s] + kv_off, stride,
                             j->pos[s] + 1u, j->head_dim, scale, vo, &m, &l);
            const float inv_l = 1.0f / l;
            for (uint32_t i = 0; i < j->head_dim; ++i) j->out[qo + i] = vo[i] * inv_l;
        }
    }
    return NULL;
}

/* ------------------------------------------------------------------------ */
/* Attention-sink eviction.  Counter-rotation of one key head by the table row
 * (c, s) of position n_discard: lfm3_counter_rotate_key_head_avx2
 * (tools/lfm2_runtime_features.c:1026-1051) and the inline AVX2 loop of
 * lfm2_kv_cache_shift_sinks_avx2 (:784-828) -- fmadd(lo, c, hi*s) and
 * fmsub(hi, c, lo*s), RNE store. */
static void orc_counter_rotate(uint16_t *kh, uint32_t head_dim, const float *c, const float *s) {
    const uint32_t half = head_dim / 2u;
    for (uint32_t i = 0; i < half; ++i) {
        const float lo = orc_f16_to_f32(kh[i]), hi = orc_f16_to_f32(kh[i + half]);
        const float hs = hi * s[i], ls = lo * s[i];
        kh[i]        = orc_f32_to_f16(fmaf(lo, c[i], hs));
        kh[i + half] = orc_f32_to_f16(fmaf(hi, c[i], -ls));
    }
}

/* Linear-cache shift of one layer: memmove of values and keys, then every
 * moved key counter-rotated (tools/lfm2_runtime_features.c:769-829). */
static void orc_shift_linear(uint16_t *kc, uint16_t *vc, size_t kv_dim, uint32_t head_dim,
                             uint32_t n_heads, uint32_t n_sink, uint32_t n_keep,
                             uint32_t n_discard, const float *c, const float *s) {
    memmove(vc + (size_t)n_sink * kv_dim, vc + (size_t)(n_sink + n_discard) * kv_dim,
            (size_t)n_keep * kv_dim * sizeof(uint16_t));
    memmove(kc + (size_t)n_sink * kv_dim, kc + (size_t)(n_sink + n_discard) * kv_dim,
            (size_t)n_keep * kv_dim * sizeof(uint16_t));
    for (uint32_t t = n_sink; t < n_sink + n_keep; ++t)
        for (uint32_t h = 0; h < n_heads; ++h)
            orc_counter_rotate(kc + (size_t)t * kv_dim + (size_t)h * head_dim, head_dim, c, s);
}

/* lfm2_kv_cache_shift_sinks_avx2, tools/lfm2_runtime_features.c:744-833. */
uint32_t orc_kv_shift_sinks_lfm2(uint16_t **k_caches, uint16_t **v_caches, uint32_t n_layers,
                                 const uint32_t *n_head_kv, uint32_t head_dim,
                                 const float *cos_lut, const float *sin_lut, uint32_t pos,
                                 uint32_t n_sink, uint32_t n_discard) {
    if (n_discard == 0u || pos <= n_sink + n_discard) return pos; /* :752 */
    if (head_dim != 64u) return pos;                                /* :755-758 */
    const uint32_t n_keep = pos - (n_sink + n_discard);
    const float *c = cos_lut + (size_t)n_discard * 32u, *s = sin_lut + (size_t)n_discard * 32u;
    for (uint32_t l = 0; l < n_layers; ++l) {
        if (!k_caches[l] || !v_caches[l] || n_head_kv[l] == 0u) continue;
        orc_shift_linear(k_caches[l], v_caches[l], (size_t)n_head_kv[l] * 64u, 64u, n_head_kv[l],
                         n_sink, n_keep, n_discard, c, s);
    }
    return n_sink + n_keep;
}

/* lfm3_kv_cache_shift_sinks, tools/lfm2_runtime_features.c:1055-1163. */
uint32_t orc_kv_shift_sinks_lfm3(uint16_t **k_caches, uint16_t **v_caches, uint32_t n_layers,
                                 const uint32_t *n_head_kv, const uint8_t *layer_kind,
                                 uint32_t head_dim, const float *cos_full, const float *sin_full,
                                 uint32_t full_rows, const float *cos_swa, const float *sin_swa,
                                 uint32_t swa_rows, uint32_t sliding_window, uint32_t swa_cap,
                                 uint32_t pos, uint32_t n_sink, uint32_t n_discard) {
    if (n_discard == 0u || pos <= n_sink + n_discard) return pos;   /* :1067 */
    if (n_discard >= full_rows || n_discard >= swa_rows) return pos; /* :1068 */
    if (head_dim % 2u != 0u) return pos;                            /* :1072 */
    const uint32_t half    = head_dim / 2u;
    const uint32_t n_keep  = pos - (n_sink + n_discard);
    const uint32_t new_pos = n_sink + n_keep;
    const uint32_t win     = sliding_window > 0u ? sliding_window : 256u;
    const uint32_t cap     = swa_cap > 0u ? swa_cap : win + 8u;
    const float *cf = cos_full + (size_t)n_discard * half, *sf = sin_full + (size_t)n_discard * half;
    const float *cw = cos_swa + (size_t)n_discard * half, *sw = sin_swa + (size_t)n_discard * half;
    for (uint32_t l = 0; l < n_layers; ++l) {
        if (layer_kind[l] == 0u || !k_caches[l] || !v_caches[l] || n_head_kv[l] == 0u) continue;
        uint16_t *kc = k_caches[l], *vc = v_caches[l];
        const size_t kv_dim = (size_t)n_head_kv[l] * head_dim;
        if (layer_kind[l] == 2u) {
            /* :1101-1135: gather the new window through temporaries, then
             * store each position at its new ring slot */
            const uint32_t t0 = new_pos > win ? new_pos - win : 0u;
            const uint32_t n_valid = new_pos - t0;
            uint16_t *tk = (uint16_t *)malloc((size_t)n_valid * kv_dim * sizeof(uint16_t));
            uint16_t *tv = (uint16_t *)malloc((size_t)n_valid * kv_dim * sizeof(uint16_t));
            if (!tk || !tv) {
                free(tk);
                free(tv);
                continue;
            }
            for (uint32_t i = 0; i < n_valid; ++i) {
                const uint32_t t = t0 + i;
                const int kept = t >= n_sink;
                const uint32_t so = (kept ? t + n_discard : t) % cap;
                memcpy(tk + (size_t)i * kv_dim, kc + (size_t)so * kv_dim, kv_dim * sizeof(uint16_t));
                memcpy(tv + (size_t)i * kv_dim, vc + (size_t)so * kv_dim, kv_dim * sizeof(uint16_t));
                if (kept)
                    for (uint32_t h = 0; h < n_head_kv[l]; ++h)
                        orc_counter_rotate(tk + (size_t)i * kv_dim + (size_t)h * head_dim, head_dim, cw, sw);
            }
            for (uint32_t i = 0; i < n_valid; ++i) {
                const uint32_t sn = (t0 + i) % cap;
                memcpy(kc + (size_t)sn * kv_dim, tk + (size_t)i * kv_dim, kv_dim * sizeof(uint16_t));
                memcpy(vc + (size_t)sn * kv_dim, tv + (size_t)i * kv_dim, kv_dim * sizeof(uint16_t));
            }
            free(tk);
            free(tv);
        } else {
            orc_shift_linear(kc, vc, kv_dim, head_dim, n_head_kv[l], n_sink, n_keep, n_discard, cf, sf);
        }
    }
    return new_pos;
}

void orc_decode_batch_mt(const float *q, const uint16_t *const *k_seq,
                         const uint16_t *const *v_seq, const uint32_t *pos,
                         float *out, uint32_t n_seq, uint32_t n_head_q,
                         uint32_t n_head_kv, uint32_t head_dim, uint32_t n_threads) {
    orc_batch_job job = {q, k_seq, v_seq, pos, out, n_seq, n_head_q, n_head_kv, head_dim,
                         (n_head_q + 3u) / 4u, 0u};
    if (n_threads < 1u) n_threads = 1u;
    if (n_threads > 256u) n_threads = 256u;
    pthread_t th[256];
    for (uint32_t t = 1; t < n_threads; ++t) pthread_create(&th[t], NULL, orc_batch_worker, &job);
    orc_batch_worker(&job);
    for (uint32_t t = 1; t < n_threads; ++t) pthread_join(th[t], NULL);
}

/* ==== next-row projections: Q8_K activations, Q4_K x Q8_K matmul ======== */

/* 6-bit scale and min of sub-block j of a Q4_K super-block
 * (get_scale_min_k4, tools/lfm2_cpuid_quants.c:180-189). */
static void q4k_scale_min(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m  = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *m  = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* packs_epi32 then packs_epi16: signed saturation to int8 */
static int8_t sat_i8(int32_t v) {
    if (v > 127) return 127;
    if (v < -128) return -128;
    return (int8_t)v;
}

void orc_quantize_q8_K(const float *x, void *y, uint32_t n_rows, uint32_t n_cols) {
    const uint32_t nb = n_cols / 256u;
    uint8_t *out = (uint8_t *)y;
    for (uint32_t t = 0; t < n_rows; ++t) {
        for (uint32_t b = 0; b < nb; ++b) {
            const float *xb = x + (size_t)t * n_cols + (size_t)b * 256u;
            uint8_t *blk    = out + ((size_t)t * nb + b) * ORC_Q8K_BYTES;
            float max_abs = 0.0f;
            for (int i = 0; i < 256; ++i) {
                const float a = fabsf(xb[i]);
                if (a > max_abs) max_abs = a;
            }
            if (max_abs == 0.0f) {
                memset(blk, 0, ORC_Q8K_BYTES);
                continue;
            }
            const float d      = max_abs / 127.0f;
            const float iscale = 127.0f / max_abs;
            memcpy(blk, &d, 4);
            for (int j = 0; j < 16; ++j) {
                int32_t bsum = 0;
                for (int l = 0; l < 16; ++l) {
                    const float p   = xb[j * 16 + l] * iscale;
                    const int32_t q = (int32_t)lrintf(p); /* round half to even */
                    blk[4 + j * 16 + l] = (uint8_t)sat_i8(q);
                    bsum += q;
                }
                const int16_t bs = (int16_t)bsum;
                memcpy(blk + 260 + 2 * j, &bs, 2);
            }
        }
    }
}

float orc_dot_q4_K_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols) {
    const uint32_t nb = n_cols / 256u;
    const uint8_t *w  = (const uint8_t *)w_row;
    const uint8_t *xq = (const uint8_t *)x_q8;
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *wb = w + (size_t)b * ORC_Q4K_BYTES;
        const uint8_t *xb = xq + (size_t)b * ORC_Q8K_BYTES;
        float d8;
        memcpy(&d8, xb, 4);
        if (d8 == 0.0f) continue;
        uint16_t dh, mh;
        memcpy(&dh, wb, 2);
        memcpy(&mh, wb + 2, 2);
        const float d    = orc_f16_to_f32(dh) * d8;
        const float dmin = orc_f16_to_f32(mh) * d8;
        const uint8_t *scales = wb + 4, *qs = wb + 16;
        const int8_t *q8      = (const int8_t *)(xb + 4);
        int16_t bs[16];
        memcpy(bs, xb + 260, sizeof bs);
        int32_t dot = 0, mins = 0;
        for (int j = 0; j < 4; ++j) { /* sub-blocks 2j (low nibbles) and 2j+1 (high) */
            int sc1, m1, sc2, m2;
            q4k_scale_min(2 * j, scales, &sc1, &m1);
            q4k_scale_min(2 * j + 1, scales, &sc2, &m2);
            mins += m1 * ((int32_t)bs[4 * j] + bs[4 * j + 1]) + m2 * ((int32_t)bs[4 * j + 2] + bs[4 * j + 3]);
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; ++l) {
                const uint8_t q = qs[32 * j + l];
                lo += (int32_t)(q & 0x0F) * q8[64 * j + l];
                hi += (int32_t)(q >> 4) * q8[64 * j + 32 + l];
            }
            dot += sc1 * lo + sc2 * hi;
        }
        const float a = d * (float)dot;
        const float m = dmin * (float)mins;
        sumf += a - m;
    }
    return sumf;
}

void orc_matmul_q4_K(float *out, const void *w, uint32_t n_rows, uint32_t n_cols,
                     const void *x_q8, uint32_t n_tokens) {
    const uint32_t nb = n_cols / 256u;
    for (uint32_t t = 0; t < n_tokens; ++t)
        for (uint32_t r = 0; r < n_rows; ++r)
            out[(size_t)t * n_rows + r] =
                orc_dot_q4_K_q8_K((const uint8_t *)w + (size_t)r * nb * ORC_Q4K_BYTES,
                                  (const uint8_t *)x_q8 + (size_t)t * nb * ORC_Q8K_BYTES, n_cols);
}

float orc_dot_q6_K_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols) {
    const uint32_t nb = n_cols / 256u;
    const uint8_t *w  = (const uint8_t *)w_row;
    const uint8_t *xq = (const uint8_t *)x_q8;
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *wb = w + (size_t)b * ORC_Q6K_BYTES;
        const uint8_t *xb = xq + (size_t)b * ORC_Q8K_BYTES;
        float d8;
        memcpy(&d8, xb, 4);
        if (d8 == 0.0f) continue;
        uint16_t dh;
        memcpy(&dh, wb + 208, 2);
        const float d = orc_f16_to_f32(dh) * d8;
        const uint8_t *ql = wb, *qh = wb + 128;
        const int8_t *sc  = (const int8_t *)(wb + 192);
        const int8_t *q8  = (const int8_t *)(xb + 4);
        int16_t bs[16];
        memcpy(bs, xb + 260, sizeof bs);
        int32_t offset = 0;
        for (int is = 0; is < 16; ++is) offset += (int32_t)sc[is] * bs[is];
        int32_t acc = 0;
        for (int half = 0; half < 2; ++half) {
            const uint8_t *l_ = ql + 64 * half, *h_ = qh + 32 * half;
            const int8_t *s_ = sc + 8 * half, *x_ = q8 + 128 * half;
            for (int l = 0; l < 32; ++l) {
                const int32_t u1 = (l_[l] & 0x0F) | ((h_[l] & 0x03) << 4);
                const int32_t u2 = (l_[l + 32] & 0x0F) | ((h_[l] & 0x0C) << 2);
                const int32_t u3 = (l_[l] >> 4) | (h_[l] & 0x30);
                const int32_t u4 = (l_[l + 32] >> 4) | ((h_[l] & 0xC0) >> 2);
                const int g = l / 16;
                acc += u1 * x_[l] * s_[g] + u2 * x_[l + 32] * s_[2 + g] + u3 * x_[l + 64] * s_[4 + g] +
                       u4 * x_[l + 96] * s_[6 + g];
            }
        }
        sumf += d * (float)(acc - 32 * offset);
    }
    return sumf;
}

/* Q4_0 (fp16 d, qs[16]: element l in the low nibble of qs[l], element l + 16
 * in the high nibble; w = d * (nibble - 8)) x Q8_K
 * (lfm2_vec_dot_q4_0_q8_K_scalar, tools/lfm2_cpuid_quants.c:252-281; the
 * AVX2 and AVX-VNNI variants at :634-672, :1659-1693 round alike): per
 * super-block, block_sum = sum over its 8 blocks in order of
 * d * (sum(u4 * q8) - 8 * (bsum[2j] + bsum[2j+1])), then sumf += d8 * block_sum. */
float orc_dot_q4_0_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols) {
    const uint32_t nb = n_cols / 256u;
    const uint8_t *w  = (const uint8_t *)w_row;
    const uint8_t *xq = (const uint8_t *)x_q8;
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *xb = xq + (size_t)b * ORC_Q8K_BYTES;
        float d8;
        memcpy(&d8, xb, 4);
        if (d8 == 0.0f) continue;
        const int8_t *q8 = (const int8_t *)(xb + 4);
        int16_t bs[16];
        memcpy(bs, xb + 260, sizeof bs);
        float block_sum = 0.0f;
        for (int j = 0; j < 8; ++j) {
            const uint8_t *blk = w + ((size_t)b * 8 + j) * ORC_Q4_0_BYTES;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            int32_t acc = 0;
            for (int l = 0; l < 16; ++l)
                acc += (int32_t)(blk[2 + l] & 0x0F) * q8[32 * j + l] + (int32_t)(blk[2 + l] >> 4) * q8[32 * j + 16 + l];
            const int32_t s8 = (int32_t)bs[2 * j] + bs[2 * j + 1];
            const float t    = orc_f16_to_f32(dh) * (float)(acc - 8 * s8);
            block_sum        = block_sum + t;
        }
        const float tb = d8 * block_sum;
        sumf           = sumf + tb;
    }
    return sumf;
}

/* Q8_0 (fp16 d, int8 qs[32]) x Q8_K (lfm2_vec_dot_q8_0_q8_K_avx2,
 * include/lfm2_simd_avx2.h:639-674; scalar tools/lfm2_cpuid_quants.c:389-410,
 * AVX-VNNI :1700-1731): the same order as Q4_0 with d * sum(q * q8). */
float orc_dot_q8_0_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols) {
    const uint32_t nb = n_cols / 256u;
    const uint8_t *w  = (const uint8_t *)w_row;
    const uint8_t *xq = (const uint8_t *)x_q8;
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *xb = xq + (size_t)b * ORC_Q8K_BYTES;
        float d8;
        memcpy(&d8, xb, 4);
        if (d8 == 0.0f) continue;
        const int8_t *q8 = (const int8_t *)(xb + 4);
        float block_sum  = 0.0f;
        for (int j = 0; j < 8; ++j) {
            const uint8_t *blk = w + ((size_t)b * 8 + j) * ORC_Q8_0_BYTES;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            int32_t acc = 0;
            for (int l = 0; l < 32; ++l) acc += (int32_t)(int8_t)blk[2 + l] * q8[32 * j + l];
            const float t = orc_f16_to_f32(dh) * (float)acc;
            block_sum     = block_sum + t;
        }
        const float tb = d8 * block_sum;
        sumf           = sumf + tb;
    }
    return sumf;
}

/* Q5_K (fp16 d, fp16 dmin, scales[12] as Q4_K, qh[32], qs[128]; element l of
 * 64-chunk c: low nibble of qs[32c + l] + 16 * bit 2c of qh[l] (sub-block
 * 2c), high nibble + 16 * bit 2c+1 (sub-block 2c+1); w = d*sc*q - dmin*m)
 * x Q8_K (lfm2_vec_dot_q5_K_q8_K_scalar, tools/lfm2_cpuid_quants.c:283-329;
 * AVX2 :690-740): sumf += (d*d8) * sum(sc*q5*q8) - (dmin*d8) * sum(m*bsum). */
float orc_dot_q5_K_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols) {
    const uint32_t nb = n_cols / 256u;
    const uint8_t *w  = (const uint8_t *)w_row;
    const uint8_t *xq = (const uint8_t *)x_q8;
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *wb = w + (size_t)b * ORC_Q5K_BYTES;
        const uint8_t *xb = xq + (size_t)b * ORC_Q8K_BYTES;
        float d8;
        memcpy(&d8, xb, 4);
        if (d8 == 0.0f) continue;
        uint16_t dh, mh;
        memcpy(&dh, wb, 2);
        memcpy(&mh, wb + 2, 2);
        const float d = orc_f16_to_f32(dh) * d8, dmin = orc_f16_to_f32(mh) * d8;
        const uint8_t *sc = wb + 4, *qh = wb + 16, *qs = wb + 48;
        const int8_t *q8 = (const int8_t *)(xb + 4);
        int16_t bs[16];
        memcpy(bs, xb + 260, sizeof bs);
        int32_t sum_q = 0, sum_m = 0;
        for (int c = 0; c < 4; ++c) {
            int32_t sc1, m1, sc2, m2;
            q4k_scale_min(2 * c, sc, &sc1, &m1);
            q4k_scale_min(2 * c + 1, sc, &sc2, &m2);
            sum_m += m1 * (bs[4 * c] + bs[4 * c + 1]) + m2 * (bs[4 * c + 2] + bs[4 * c + 3]);
            int32_t s1 = 0, s2 = 0;
            for (int l = 0; l < 32; ++l) {
                const int32_t lo = (qs[32 * c + l] & 0x0F) + (((qh[l] >> (2 * c)) & 1) << 4);
                const int32_t hi = (qs[32 * c + l] >> 4) + (((qh[l] >> (2 * c + 1)) & 1) << 4);
                s1 += lo * q8[64 * c + l];
                s2 += hi * q8[64 * c + 32 + l];
            }
            sum_q += sc1 * s1 + sc2 * s2;
        }
        const float ta = d * (float)sum_q, tm = dmin * (float)sum_m;
        const float tb = ta - tm;
        sumf           = sumf + tb;
    }
    return sumf;
}

/* IQ4_XS (fp16 d, scales_h (2 high bits of 8 6-bit scales), scales_l[4] (low
 * 4 bits), qs[128]; sub-block ib: 16 bytes, element j the low nibble, j + 16
 * the high nibble, both indices into the fixed IQ4_NL grid; scale
 * ls = 6-bit - 32) x Q8_K (lfm2_vec_dot_iq4_xs_q8_K_scalar,
 * tools/lfm2_cpuid_quants.c:336-364; AVX2 :832-880): sumf += (d*d8) * sum(ls * dot). */
static const int8_t k_iq4nl_grid[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                        1,    13,   25,  38,  53,  69,  89,  113};

float orc_dot_iq4_xs_q8_K(const void *w_row, const void *x_q8, uint32_t n_cols) {
    const uint32_t nb = n_cols / 256u;
    const uint8_t *w  = (const uint8_t *)w_row;
    const uint8_t *xq = (const uint8_t *)x_q8;
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *wb = w + (size_t)b * ORC_IQ4XS_BYTES;
        const uint8_t *xb = xq + (size_t)b * ORC_Q8K_BYTES;
        float d8;
        memcpy(&d8, xb, 4);
        if (d8 == 0.0f) continue;
        uint16_t dh, sh;
        memcpy(&dh, wb, 2);
        memcpy(&sh, wb + 2, 2);
        const uint8_t *sl = wb + 4, *qs = wb + 8;
        const int8_t *q8 = (const int8_t *)(xb + 4);
        int32_t acc = 0;
        for (int ib = 0; ib < 8; ++ib) {
            const int32_t ls = (((sl[ib >> 1] >> (4 * (ib & 1))) & 0x0F) | (((sh >> (2 * ib)) & 3) << 4)) - 32;
            int32_t dot = 0;
            for (int j = 0; j < 16; ++j)
                dot += k_iq4nl_grid[qs[16 * ib + j] & 0x0F] * q8[32 * ib + j] +
                       k_iq4nl_grid[qs[16 * ib + j] >> 4] * q8[32 * ib + 16 + j];
            acc += ls * dot;
        }
        const float d  = orc_f16_to_f32(dh) * d8;
        const float tb = d * (float)acc;
        sumf           = sumf + tb;
    }
    return sumf;
}

size_t orc_q_row_bytes(uint32_t type, uint32_t n_cols) {
    const size_t nb = n_cols / 256u;
    switch (type) {
    case 2u: return nb * 8u * ORC_Q4_0_BYTES;
    case 8u: return nb * 8u * ORC_Q8_0_BYTES;
    case 12u: return nb * ORC_Q4K_BYTES;
    case 13u: return nb * ORC_Q5K_BYTES;
    case 14u: return nb * ORC_Q6K_BYTES;
    case 23u: return nb * ORC_IQ4XS_BYTES;
    default: return 0;
    }
}

void orc_matmul_q(float *out, const void *w, uint32_t type, uint32_t n_rows, uint32_t n_cols,
                  const void *x_q8, uint32_t n_tokens) {
    const uint32_t nb = n_cols / 256u;
    const size_t rowb = orc_q_row_bytes(type, n_cols);
    float (*dot)(const void *, const void *, uint32_t) =
        type == 2u ? orc_dot_q4_0_q8_K : type == 8u ? orc_dot_q8_0_q8_K : type == 13u ? orc_dot_q5_K_q8_K
        : type == 14u ? orc_dot_q6_K_q8_K : type == 23u ? orc_dot_iq4_xs_q8_K : orc_dot_q4_K_q8_K;
    for (uint32_t t = 0; t < n_tokens; ++t)
        for (uint32_t r = 0; r < n_rows; ++r) {
            const void *wr = (const uint8_t *)w + (size_t)r * rowb;
            const void *xt = (const uint8_t *)x_q8 + (size_t)t * nb * ORC_Q8K_BYTES;
            out[(size_t)t * n_rows + r] = dot(wr, xt, n_cols);
        }
}
