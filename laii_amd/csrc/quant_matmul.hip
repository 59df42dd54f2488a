/*
 * quant_matmul.hip -- the projections beside the attention path on gfx950:
 * Q8_K quantization of activations and the Q4_K x Q8_K matrix-vector /
 * small-batch product (`wo` after attention, fused Q/K/V before it).
 *
 * Formats are the reference's packed GGUF blocks
 * (tools/lfm2_cpuid_quants.c:76-127):
 *   block_q4_K, 144 B: fp16 d, fp16 dmin, scales[12], qs[128].  Sub-block j
 *     (32 weights) has a 6-bit scale and min packed in scales[]; its weights
 *     are the low (even j) or high (odd j) nibbles of qs[32*(j/2) .. +32]:
 *     w = d*sc*q - dmin*m.
 *   block_q8_K, 292 B: float d, int8 qs[256], int16 bsums[16] (sums of 16
 *     consecutive qs): x = d*q.
 *
 * Arithmetic follows the reference exactly where it is exact, and in its
 * order where it rounds:
 *   quantize  d = max|x| / 127, iscale = 127 / max|x| (correctly rounded),
 *             q = round-half-even(x * iscale), bsums of the unsaturated q
 *             (lfm2_quantize_row_q8_K_avx2_cpuid, tools/lfm2_cpuid_quants.c:585-635);
 *   dot       per super-block the integer sums sum(sc*q4*q8) and
 *             sum(m*bsum) (exact), then sumf += (d*d8)*dot - (dmin*d8)*mins
 *             with every product and sum rounded separately, super-blocks in
 *             order (lfm2_vec_dot_q4_K_q8_K_avx2, include/lfm2_simd_avx2.h:364-412).
 * So results are bit-identical to that reference kernel.
 *
 * Work decomposition of the product: one wave per R consecutive rows; the 8
 * lanes of a lane group take the 8 16-byte parts of one super-block's qs
 * (part p holds 16 weights of sub-block 2*(p/2) in its low nibbles and 16 of
 * sub-block 2*(p/2)+1 in its high nibbles), so a wave covers 8 super-blocks
 * (2048 columns) per step, reading each weight byte once.  Integer dots use
 * v_dot4_i32_i8; the lane groups' sums meet by shuffles.  The product is
 * HBM-bound on the weights (4.5 bits per weight).
 */
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "lfm_attn.h"

namespace lfm {
namespace {

constexpr uint32_t kQ4K = 144u, kQ8K = 292u;
constexpr int kRows = 4; /* rows per wave */

__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

/* ---- Q8_K quantization: one wave per 256-value block ----------------------- */
__global__ __launch_bounds__(256) void k_quant_q8K(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                   uint32_t n_blocks, uint32_t nb) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t blk  = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (blk >= n_blocks) return;
    const uint32_t t = blk / nb, b = blk - t * nb;
    const float *xb = x + ((size_t)t * nb + b) * 256u + 4u * lane;
    const float v[4] = {xb[0], xb[1], xb[2], xb[3]};
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    uint8_t *out = y + (size_t)blk * kQ8K;
    if (amax == 0.0f) {
        *reinterpret_cast<uint32_t *>(out + 4u + 4u * lane) = 0u;
        if (lane < 16u) *reinterpret_cast<int16_t *>(out + 260u + 2u * lane) = 0;
        if (lane == 0u) *reinterpret_cast<float *>(out) = 0.0f;
        return;
    }
    const float d      = amax / 127.0f;  /* correctly rounded (HIP default) */
    const float iscale = 127.0f / amax;
    int32_t q[4], part = 0;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        q[i] = (int32_t)__builtin_rintf(v[i] * iscale); /* one rounding, then half-even */
        part += q[i];
        const int32_t s = q[i] > 127 ? 127 : (q[i] < -128 ? -128 : q[i]);
        packed |= (uint32_t)(uint8_t)(int8_t)s << (8 * i);
    }
    *reinterpret_cast<uint32_t *>(out + 4u + 4u * lane) = packed;
    part += __shfl_xor(part, 1);
    part += __shfl_xor(part, 2);
    if ((lane & 3u) == 0u) *reinterpret_cast<int16_t *>(out + 260u + (lane >> 1)) = (int16_t)part;
    if (lane == 0u) *reinterpret_cast<float *>(out) = d;
}

/* 6-bit scale and min of sub-block j (get_scale_min_k4,
 * tools/lfm2_cpuid_quants.c:180-189); sc12 holds the 12 scale bytes. */
__device__ __forceinline__ void scale_min(uint32_t j, const uint8_t *sc12, int32_t *sc, int32_t *m) {
    if (j < 4u) {
        *sc = sc12[j] & 63;
        *m  = sc12[j + 4u] & 63;
    } else {
        *sc = (sc12[j + 4u] & 0x0F) | ((sc12[j - 4u] >> 6) << 4);
        *m  = (sc12[j + 4u] >> 4) | ((sc12[j] >> 6) << 4);
    }
}

/* One super-block's term: (d*d8)*dot - (dmin*d8)*mins, each step rounded. */
__device__ __forceinline__ float block_term(float d, float dmin, float d8, int32_t dot, int32_t mins) {
#pragma clang fp contract(off)
    const float dd = d * d8, dm = dmin * d8;
    return dd * (float)dot - dm * (float)mins;
}

__device__ __forceinline__ float add_rounded(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}

/* ---- Q4_K x Q8_K: out[t][r] --------------------------------------------------- */
__global__ __launch_bounds__(256) void k_matmul_q4K(float *__restrict__ out, const uint8_t *__restrict__ w,
                                                    const uint8_t *__restrict__ xq, uint32_t n_rows,
                                                    uint32_t nb, uint32_t n_tokens) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t r0   = (blockIdx.x * 4u + (threadIdx.x >> 6)) * kRows;
    if (r0 >= n_rows) return;
    const uint32_t p  = lane & 7u;  /* 16-byte part of qs              */
    const uint32_t g  = lane >> 3;  /* super-block slot of this step   */
    const uint32_t jp = p >> 1;     /* sub-block pair                  */
    const uint32_t h  = p & 1u;     /* first or second 16 of each half */
    /* q8 offsets of this part's 16 low-nibble and 16 high-nibble partners */
    const uint32_t qlo = 4u + 64u * jp + 16u * h, qhi = qlo + 32u;
    const uint32_t bslo = 260u + 2u * (4u * jp + h), bshi = bslo + 4u;
    const size_t row_bytes = (size_t)nb * kQ4K;

    for (uint32_t t = 0; t < n_tokens; ++t) {
        const uint8_t *xt = xq + (size_t)t * nb * kQ8K;
        float sumf[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) sumf[r] = 0.0f;
        for (uint32_t b0 = 0; b0 < nb; b0 += 8u) {
            const uint32_t b   = b0 + g;
            const bool live    = b < nb;
            const uint8_t *xb  = xt + (size_t)(live ? b : 0u) * kQ8K;
            const float d8     = *reinterpret_cast<const float *>(xb);
            uint32_t xl[4], xh[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xl[i] = ld32(xb + qlo + 4u * i);
                xh[i] = ld32(xb + qhi + 4u * i);
            }
            const int32_t bsl = *reinterpret_cast<const int16_t *>(xb + bslo);
            const int32_t bsh = *reinterpret_cast<const int16_t *>(xb + bshi);
            float term[kRows];
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const uint32_t row = min(r0 + (uint32_t)r, n_rows - 1u);
                const uint8_t *wb  = w + row * row_bytes + (size_t)(live ? b : 0u) * kQ4K;
                const uint4 hdr    = *reinterpret_cast<const uint4 *>(wb);
                const uint4 qs     = *reinterpret_cast<const uint4 *>(wb + 16u + 16u * p);
                uint8_t sc12[12];
                __builtin_memcpy(sc12, reinterpret_cast<const uint8_t *>(&hdr) + 4, 12);
                int32_t sc1, m1, sc2, m2;
                scale_min(2u * jp, sc12, &sc1, &m1);
                scale_min(2u * jp + 1u, sc12, &sc2, &m2);
                const uint32_t qv[4] = {qs.x, qs.y, qs.z, qs.w};
                int32_t lo = 0, hi = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lo = __builtin_amdgcn_sdot4((int)(qv[i] & 0x0F0F0F0Fu), (int)xl[i], lo, false);
                    hi = __builtin_amdgcn_sdot4((int)((qv[i] >> 4) & 0x0F0F0F0Fu), (int)xh[i], hi, false);
                }
                int32_t dot  = sc1 * lo + sc2 * hi;
                int32_t mins = m1 * bsl + m2 * bsh;
#pragma unroll
                for (int o = 1; o < 8; o <<= 1) {
                    dot += __shfl_xor(dot, o);
                    mins += __shfl_xor(mins, o);
                }
                const float d    = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu));
                const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
                term[r]          = block_term(d, dmin, d8, dot, mins);
            }
            /* super-blocks b0 .. b0+7 in order; a block whose d8 is 0 adds nothing */
#pragma unroll
            for (uint32_t i = 0; i < 8u; ++i) {
                if (b0 + i >= nb) break;
                const float d8i = __shfl(d8, (int)(8u * i));
#pragma unroll
                for (int r = 0; r < kRows; ++r) {
                    const float ti = __shfl(term[r], (int)(8u * i));
                    if (d8i != 0.0f) sumf[r] = add_rounded(sumf[r], ti);
                }
            }
        }
        if (lane < (uint32_t)kRows && r0 + lane < n_rows) {
            float v = sumf[0];
#pragma unroll
            for (int r = 1; r < kRows; ++r)
                if (lane == (uint32_t)r) v = sumf[r];
            out[(size_t)t * n_rows + r0 + lane] = v;
        }
    }
}

} // namespace

int launch_quantize_q8_K(const float *x, void *y, uint32_t n_rows, uint32_t n_cols, hipStream_t stream) {
    const uint32_t nb       = n_cols / 256u;
    const uint64_t n_blocks = (uint64_t)n_rows * nb;
    if (n_blocks == 0u) return LFM_ATTN_OK;
    hipLaunchKernelGGL(k_quant_q8K, dim3((uint32_t)((n_blocks + 3u) / 4u)), dim3(256), 0, stream, x,
                       static_cast<uint8_t *>(y), (uint32_t)n_blocks, nb);
    return hip_status(hipGetLastError());
}

int launch_matmul_q4_K(float *out, const void *w, uint32_t n_rows, uint32_t n_cols, const void *x_q8,
                       uint32_t n_tokens, hipStream_t stream) {
    if (n_rows == 0u || n_tokens == 0u) return LFM_ATTN_OK;
    const uint32_t waves = (n_rows + kRows - 1u) / kRows;
    hipLaunchKernelGGL(k_matmul_q4K, dim3((waves + 3u) / 4u), dim3(256), 0, stream, out,
                       static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(x_q8), n_rows,
                       n_cols / 256u, n_tokens);
    return hip_status(hipGetLastError());
}

} // namespace lfm
