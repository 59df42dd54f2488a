/*
 * prologue.hip -- per-head QK-RMSNorm + NeoX RoPE and the RNE fp16 KV stores
 * that precede every attention call in the reference forward stacks.
 *
 *   lfm2_qk_norm_rope_avx2 / _scalar   tools/lfm2_kernels_fast.c:403-497, 511-547
 *   lfm3_qk_norm_rope_128_avx2 / _scalar tools/lfm3_engine.c:463-525, 599-642
 *   lfm2_store_fp32_to_fp16_*          tools/lfm2_kernels_fast.c:500-507, 549-555
 *   batched per-token prologue         tools/lfm2_prefill_batch.c:1029-1072,
 *                                      tools/lfm3_engine.c:2006-2016
 *
 * Per head: irms = 1/sqrtf(sum(x^2)/head_dim + eps), the sum added in the
 * AVX2 kernels' order at head_dim 64 and 128 (LFM_PROLOGUE_FAST) or in
 * lfm2_rmsnorm's order (LFM_PROLOGUE_TABLE, the prologue of
 * tools/lfm2_forward.c:775-830 and tools/lfm2_prefill_batch.c:826-893,
 * any head_dim); x <- (x*irms)*w (skipped
 * when w is NULL); pairs (i, i+head_dim/2) rotate by the LUT row of the
 * position: lo' = lo*c - hi*s, hi' = hi*c + lo*s (fused multiply-add, as the
 * AVX2 kernels do).  fp16 stores round to nearest even.  One wave64 per head;
 * lane j owns the pairs j and j+64.
 */
#include <hip/hip_runtime.h>

#include "attn_index.h"
#include "kernels.h"
#include "lfm_attn.h"

namespace lfm {
namespace {

__device__ __forceinline__ uint16_t f16_rne(float x) {
    /* x is first rounded to fp32 (the reference stores an fp32 result with
     * _mm256_cvtps_ph): the barrier keeps the compiler from fusing a
     * producing fma with this conversion into v_fma_mixlo_f16, whose single
     * rounding differs from fp32-then-fp16 on ties */
    asm volatile("" : "+v"(x));
    return __builtin_bit_cast(uint16_t, (_Float16)x); /* v_cvt_f16_f32, round-to-nearest-even */
}

__device__ __forceinline__ float wave_sum_uniform(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

/* Sum of squares of the head at `in` for head_dim 64 or 128, added in the
 * order of the reference's AVX2 kernels (lanes 0..7 play its eight vector
 * columns), so normalised rows are bit-identical to theirs:
 *   64  lfm2_qk_norm_rope_avx2 (tools/lfm2_kernels_fast.c:443-449):
 *       ss0 = x[j]^2 + x[32+j]^2, ss1 = x[8+j]^2 + x[40+j]^2,
 *       ss0 = fma(x[16+j], ., fma(x[48+j], ., ss0)), ss1 likewise (24, 56),
 *       t = ss0 + ss1, total ((t0+t4) + (t2+t6)) + ((t1+t5) + (t3+t7));
 *   128 lfm3_qk_norm_rope_128_avx2 (tools/lfm3_engine.c:480-494):
 *       fma chains over dims 16k + j and 16k + 8 + j, s = ss0 + ss1,
 *       total ((s0+s4) + (s1+s5)) + ((s2+s6) + (s3+s7)).
 * Returned on every lane. */
__device__ __forceinline__ float sumsq_ref_order(const float *in, uint32_t hd) {
#pragma clang fp contract(off)
    const uint32_t j = threadIdx.x & 7u;
    float t;
    if (hd == 64u) {
        float ss0 = in[j] * in[j] + in[32u + j] * in[32u + j];
        float ss1 = in[8u + j] * in[8u + j] + in[40u + j] * in[40u + j];
        ss0 = __builtin_fmaf(in[16u + j], in[16u + j], __builtin_fmaf(in[48u + j], in[48u + j], ss0));
        ss1 = __builtin_fmaf(in[24u + j], in[24u + j], __builtin_fmaf(in[56u + j], in[56u + j], ss1));
        t = ss0 + ss1;
        t = t + __shfl_xor(t, 4); /* j < 4: t_j + t_(j+4)        */
        t = t + __shfl_xor(t, 2); /* (t0+t4) + (t2+t6), ...      */
        t = t + __shfl_xor(t, 1);
    } else {
        float ss0 = 0.0f, ss1 = 0.0f;
        for (uint32_t i = 0; i < 128u; i += 16u) {
            ss0 = __builtin_fmaf(in[i + j], in[i + j], ss0);
            ss1 = __builtin_fmaf(in[i + 8u + j], in[i + 8u + j], ss1);
        }
        t = ss0 + ss1;
        t = t + __shfl_xor(t, 4); /* j < 4: s_j + s_(j+4)        */
        t = t + __shfl_xor(t, 1); /* (s0+s4) + (s1+s5), ...      */
        t = t + __shfl_xor(t, 2);
    }
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, t)));
}

/* Mean of squares of the head at `in` in the order of lfm2_rmsnorm
 * (tools/lfm2_forward.c:669-684), the norm of LFM_PROLOGUE_TABLE: lane j < 8
 * is the fused multiply-add chain over dims 8k + j of every full group of
 * eight, the eight chains are added in order in double, then the dims past
 * the last full group one at a time (exact double products); the result is
 * (float)(sum / hd).  Returned on every lane. */
__device__ __forceinline__ float meansq_table_order(const float *in, uint32_t hd) {
#pragma clang fp contract(off)
    const uint32_t j    = threadIdx.x & 7u;
    const uint32_t full = hd & ~7u;
    float col = 0.0f;
    for (uint32_t d = 0; d < full; d += 8u) col = __builtin_fmaf(in[d + j], in[d + j], col);
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < 8; ++c) ss += (double)__shfl(col, c);
    for (uint32_t d = full; d < hd; ++d) ss += (double)in[d] * (double)in[d];
    return (float)(ss / (double)hd);
}

/* a*b - c*d and a*b + c*d with every product rounded on its own */
__device__ __forceinline__ float diff_of_products(float a, float b, float c, float d) {
#pragma clang fp contract(off)
    return a * b - c * d;
}
__device__ __forceinline__ float sum_of_products(float a, float b, float c, float d) {
#pragma clang fp contract(off)
    return a * b + c * d;
}

/* Normalise + rotate one head held as pairs; writes fp32 (vec_out) or fp16.
 * LFM_PROLOGUE_TABLE rotates pairs of full groups of eight with fused
 * multiply-adds and the rest with separately rounded products, as the AVX2
 * loop and scalar tail of lfm2_qk_norm_and_rope_table do
 * (tools/lfm2_prefill_batch.c:842-879). */
__device__ __forceinline__ void norm_rope_head(const float *in, float *vec_out, uint16_t *dst_f16,
                                               uint32_t hd, const float *norm_w, float eps,
                                               const float *cos_row, const float *sin_row, int prologue) {
    const uint32_t half = hd / 2u;
    const uint32_t lane = threadIdx.x;
    float x0[2], x1[2];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t i = lane + 64u * j;
        x0[j] = i < half ? in[i] : 0.0f;
        x1[j] = i < half ? in[i + half] : 0.0f;
        ss += x0[j] * x0[j] + x1[j] * x1[j];
    }
    if (norm_w) {
        const float mean = prologue == LFM_PROLOGUE_TABLE ? meansq_table_order(in, hd)
                         : ((hd == 64u || hd == 128u) ? sumsq_ref_order(in, hd) : wave_sum_uniform(ss)) / (float)hd;
        const float irms = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t i = lane + 64u * j;
            if (i < half) {
                x0[j] = (x0[j] * irms) * norm_w[i];
                x1[j] = (x1[j] * irms) * norm_w[i + half];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t i = lane + 64u * j;
        if (i >= half) continue;
        const float c = cos_row[i], s = sin_row[i];
        const bool fused = prologue != LFM_PROLOGUE_TABLE || i < (half & ~7u);
        const float r0 = fused ? __builtin_fmaf(x0[j], c, -(x1[j] * s)) : diff_of_products(x0[j], c, x1[j], s);
        const float r1 = fused ? __builtin_fmaf(x1[j], c, x0[j] * s) : sum_of_products(x1[j], c, x0[j], s);
        if (dst_f16) {
            dst_f16[i]        = f16_rne(r0);
            dst_f16[i + half] = f16_rne(r1);
        } else {
            vec_out[i]        = r0;
            vec_out[i + half] = r1;
        }
    }
}

__global__ __launch_bounds__(64) void k_qk_norm_rope(float *vec, uint16_t *dst_f16, uint32_t hd,
                                                     const float *norm_w, float eps,
                                                     const float *cos_row, const float *sin_row, int prologue) {
    const size_t off = (size_t)blockIdx.x * hd;
    norm_rope_head(vec + off, vec + off, dst_f16 ? dst_f16 + off : nullptr, hd, norm_w, eps,
                   cos_row, sin_row, prologue);
}

__global__ __launch_bounds__(256) void k_store_f16(uint16_t *dst, const float *src, uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) dst[i] = f16_rne(src[i]);
}

struct PrologueParams {
    float *q;
    const float *k;
    const float *v;
    uint16_t *const *k_seq;
    uint16_t *const *v_seq;
    const uint32_t *pos_0;
    const float *q_norm_w;
    const float *k_norm_w;
    const float *cos_lut;
    const float *sin_lut;
    uint32_t n_rows, n_head_q, n_head_kv, head_dim, window, cap;
    float eps;
    int prologue;
};

/* blockIdx.x < n_head_q: query head, rotated in place.  Otherwise KV head
 * j = blockIdx.x - n_head_q: K rotated into the fp16 cache slot, V stored. */
__global__ __launch_bounds__(64) void k_qkv_prologue(const PrologueParams P) {
    const uint32_t b = blockIdx.x, r = blockIdx.y, s = blockIdx.z;
    const uint32_t hd   = P.head_dim;
    const uint32_t pos  = P.pos_0[s] + r;
    const uint32_t half = hd / 2u;
    const float *cos_row = P.cos_lut + (size_t)pos * half;
    const float *sin_row = P.sin_lut + (size_t)pos * half;
    if (b < P.n_head_q) {
        float *qh = P.q + (((size_t)s * P.n_rows + r) * P.n_head_q + b) * hd;
        norm_rope_head(qh, qh, nullptr, hd, P.q_norm_w, P.eps, cos_row, sin_row, P.prologue);
        return;
    }
    const uint32_t j    = b - P.n_head_q;
    const uint32_t slot = lfm_slot_of(pos, P.window, P.cap);
    const size_t kv_dim = (size_t)P.n_head_kv * hd;
    const size_t src    = (((size_t)s * P.n_rows + r) * P.n_head_kv + j) * hd;
    uint16_t *kd = P.k_seq[s] + (size_t)slot * kv_dim + (size_t)j * hd;
    uint16_t *vd = P.v_seq[s] + (size_t)slot * kv_dim + (size_t)j * hd;
    norm_rope_head(P.k + src, nullptr, kd, hd, P.k_norm_w, P.eps, cos_row, sin_row, P.prologue);
    for (uint32_t i = threadIdx.x; i < hd; i += 64u) vd[i] = f16_rne(P.v[src + i]);
}

/* Gen-1 (src/lfm_forward.c:184-202): per head lfm_vec_rmsnorm_f32
 * (src/lfm_simd.c:125-174) then lfm_rope_neox (:97-111).  The sum of
 * squares follows the AVX2 kernel: eight vector columns j accumulate
 * fma(x, x, .) over dims 32b + j, 32b + 8 + j, 32b + 16 + j, 32b + 24 + j of
 * each full 32-block b; hsum256_ps adds columns k and k + 4, then the four
 * results in sequence; dims past the last full block are added one at a time
 * (product, then sum).  x <- (x * r) * w, r = 1/sqrtf(sum/n + eps); the
 * rotation uses separately rounded products (lo*c - hi*s, hi*c + lo*s) with
 * the row of lfm_attn_rope_row_gen1.  Q is rotated in place; K goes to the
 * FP32 cache row at pos, V is copied there unchanged. */
__device__ __forceinline__ void gen1_norm_rope(const float *in, float *dst, uint32_t hd, const float *norm_w,
                                               float eps, const float *cos_row, const float *sin_row) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x;
    float col = 0.0f;
    const uint32_t full = hd & ~31u;
    if (lane < 8u)
        for (uint32_t b = 0; b < full; b += 32u)
#pragma unroll
            for (uint32_t q = 0; q < 4u; ++q) col = __builtin_fmaf(in[b + 8u * q + lane], in[b + 8u * q + lane], col);
    const float pair = col + __shfl_xor(col, 4); /* columns k + k + 4 on lanes 0..3 */
    const float c1 = __shfl(pair, 1), c2 = __shfl(pair, 2), c3 = __shfl(pair, 3);
    float sum = ((pair + c1) + c2) + c3;         /* lane 0 */
    if (lane == 0u)
        for (uint32_t i = full; i < hd; ++i) sum = sum + in[i] * in[i];
    sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sum)));
    const float r    = 1.0f / sqrtf(sum / (float)hd + eps);
    const uint32_t half = hd / 2u;
    for (uint32_t i = lane; i < half; i += 64u) {
        float x0 = in[i] * r, x1 = in[i + half] * r;
        if (norm_w) {
            x0 = x0 * norm_w[i];
            x1 = x1 * norm_w[i + half];
        }
        const float c = cos_row[i], s = sin_row[i];
        dst[i]        = x0 * c - x1 * s;
        dst[i + half] = x1 * c + x0 * s;
    }
}

struct Gen1Params {
    float *q;
    const float *k;
    const float *v;
    float *k_cache;
    float *v_cache;
    const float *q_norm_w;
    const float *k_norm_w;
    const float *cos_row;
    const float *sin_row;
    uint32_t n_head_q, n_head_kv, head_dim, pos;
    float eps;
};

/* blockIdx.x < n_head_q: query head (in place); otherwise KV head. */
__global__ __launch_bounds__(64) void k_gen1_prologue(const Gen1Params P) {
    const uint32_t b = blockIdx.x, hd = P.head_dim;
    if (b < P.n_head_q) {
        float *qh = P.q + (size_t)b * hd;
        gen1_norm_rope(qh, qh, hd, P.q_norm_w, P.eps, P.cos_row, P.sin_row);
        return;
    }
    const uint32_t j   = b - P.n_head_q;
    const size_t dst   = (size_t)P.pos * P.n_head_kv * hd + (size_t)j * hd;
    gen1_norm_rope(P.k + (size_t)j * hd, P.k_cache + dst, hd, P.k_norm_w, P.eps, P.cos_row, P.sin_row);
    for (uint32_t i = threadIdx.x; i < hd; i += 64u) P.v_cache[dst + i] = P.v[(size_t)j * hd + i];
}

} // namespace

int launch_gen1_prologue(float *q, const float *k, const float *v, float *k_cache, float *v_cache,
                         const float *q_norm_w, const float *k_norm_w, float eps, const float *cos_row,
                         const float *sin_row, uint32_t pos, uint32_t n_head_q, uint32_t n_head_kv,
                         uint32_t head_dim, hipStream_t stream) {
    Gen1Params P{q, k, v, k_cache, v_cache, q_norm_w, k_norm_w, cos_row, sin_row, n_head_q, n_head_kv, head_dim,
                 pos, eps};
    hipLaunchKernelGGL(k_gen1_prologue, dim3(n_head_q + n_head_kv), dim3(64), 0, stream, P);
    return hip_status(hipGetLastError());
}

int launch_qk_norm_rope(float *vec, uint16_t *dst_f16, uint32_t n_heads, uint32_t head_dim,
                        const float *norm_w, float eps, const float *cos_lut,
                        const float *sin_lut, uint32_t pos, int prologue, hipStream_t stream) {
    const size_t row = (size_t)pos * (head_dim / 2u);
    hipLaunchKernelGGL(k_qk_norm_rope, dim3(n_heads), dim3(64), 0, stream, vec, dst_f16, head_dim,
                       norm_w, eps, cos_lut + row, sin_lut + row, prologue);
    return hip_status(hipGetLastError());
}

int launch_store_f16(uint16_t *dst, const float *src, uint32_t n, hipStream_t stream) {
    hipLaunchKernelGGL(k_store_f16, dim3((n + 255u) / 256u), dim3(256), 0, stream, dst, src, n);
    return hip_status(hipGetLastError());
}

int launch_qkv_prologue(float *q, const float *k, const float *v, uint16_t *const *k_seq,
                        uint16_t *const *v_seq, const uint32_t *pos_0, uint32_t n_seq,
                        uint32_t n_rows, uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                        const float *q_norm_w, const float *k_norm_w, float eps,
                        const float *cos_lut, const float *sin_lut, uint32_t window_len,
                        uint32_t cap, int prologue, hipStream_t stream) {
    PrologueParams P{q, k, v, k_seq, v_seq, pos_0, q_norm_w, k_norm_w, cos_lut, sin_lut,
                     n_rows, n_head_q, n_head_kv, head_dim, window_len, cap, eps, prologue};
    hipLaunchKernelGGL(k_qkv_prologue, dim3(n_head_q + n_head_kv, n_rows, n_seq), dim3(64), 0,
                       stream, P);
    return hip_status(hipGetLastError());
}

} // namespace lfm
