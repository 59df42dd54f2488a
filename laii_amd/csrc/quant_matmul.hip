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
 * Work decomposition of the product: one wave per RPW consecutive rows; the 8
 * lanes of a lane group take the 8 16-byte parts of one super-block's qs
 * (part p holds 16 weights of sub-block 2*(p/2) in its low nibbles and 16 of
 * sub-block 2*(p/2)+1 in its high nibbles), so a wave covers 8 super-blocks
 * (2048 columns) per step, reading each weight byte once.  Integer dots use
 * v_dot4_i32_i8; the lane groups' sums meet by shuffles.  The product is
 * HBM-bound on the weights (4.5 bits per weight).  Eight or more tokens on one
 * Q4_K or Q5_K matrix take k_matmul_qk_mfma instead (int8 MFMA, same
 * arithmetic).
 */
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "lfm_attn.h"

namespace lfm {
namespace {

constexpr uint32_t kQ4K = 144u, kQ8K = 292u;

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
 * tools/lfm2_cpuid_quants.c:180-189) from the 12 scale bytes held as the
 * words y (bytes 0-3), z (4-7) and w (8-11) of the block header.  Bytes are
 * picked by shifts, so a lane-dependent j needs no byte array in scratch. */
__device__ __forceinline__ void scale_min(uint32_t j, uint32_t y, uint32_t z, uint32_t w, int32_t *sc, int32_t *m) {
    const uint32_t sh = 8u * (j & 3u);
    const uint32_t b0 = (y >> sh) & 0xFFu, b4 = (z >> sh) & 0xFFu, b8 = (w >> sh) & 0xFFu;
    if (j < 4u) {
        *sc = (int32_t)(b0 & 63u);
        *m  = (int32_t)(b4 & 63u);
    } else {
        *sc = (int32_t)((b8 & 0x0Fu) | ((b0 >> 6) << 4));
        *m  = (int32_t)((b8 >> 4) | ((b4 >> 6) << 4));
    }
}

__device__ __forceinline__ float fp16_bits(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

__device__ __forceinline__ float add_rounded(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}

__device__ __forceinline__ float mul_rounded(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}

__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

/* 4 bytes from a 2-byte aligned address */
__device__ __forceinline__ uint32_t ld16x2(const uint8_t *p) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}

/* Per weight type: what lane p (0..7) of a super-block's lane group loads and
 * computes.  Both give two exact integer partials (a, b) that sum over the
 * 8 lanes, and the super-block's fp32 term in the reference's rounding order. */
template <int TYPE> struct QType;

/* Integer-partial types (Q4_K, Q5_K, Q6_K, IQ4_XS) combine their exact lane
 * sums in one fp32 term per super-block; the 32-weight block types (Q4_0,
 * Q8_0) give a float per lane (one block each) that the reference sums in
 * block order before scaling by d8 (kFloatParts). */
/* Q4_K: part p = qs bytes 16p..16p+15: 16 weights of sub-block 2*(p/2) (low
 * nibbles) and of sub-block 2*(p/2)+1 (high nibbles); a = sum(sc*q4*q8),
 * b = sum(m*bsum); term = (d*d8)*a - (dmin*d8)*b
 * (include/lfm2_simd_avx2.h:364-412). */
template <> struct QType<12> {
    static constexpr uint32_t kBytes = 144u;
    static constexpr bool kFloatParts = false;
    struct W { uint32_t q[4]; int32_t sc1, m1, sc2, m2; float d, dmin; };
    struct X { float d8; uint32_t lo[4], hi[4]; int32_t bl, bh; };
    static __device__ __forceinline__ void load_w(W &w, const uint8_t *blk, uint32_t p) {
        const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qs  = *reinterpret_cast<const uint4 *>(blk + 16u + 16u * p);
        w.q[0] = qs.x;
        w.q[1] = qs.y;
        w.q[2] = qs.z;
        w.q[3] = qs.w;
        scale_min(2u * (p >> 1), hdr.y, hdr.z, hdr.w, &w.sc1, &w.m1);
        scale_min(2u * (p >> 1) + 1u, hdr.y, hdr.z, hdr.w, &w.sc2, &w.m2);
        w.d    = fp16_bits(hdr.x & 0xFFFFu);
        w.dmin = fp16_bits(hdr.x >> 16);
    }
    static __device__ __forceinline__ void load_x(X &x, const uint8_t *xb, uint32_t p) {
        const uint32_t jp = p >> 1, h = p & 1u;
        const uint32_t qlo = 4u + 64u * jp + 16u * h, qhi = qlo + 32u;
        x.d8 = *reinterpret_cast<const float *>(xb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x.lo[i] = ld32(xb + qlo + 4u * i);
            x.hi[i] = ld32(xb + qhi + 4u * i);
        }
        x.bl = *reinterpret_cast<const int16_t *>(xb + 260u + 2u * (4u * jp + h));
        x.bh = *reinterpret_cast<const int16_t *>(xb + 260u + 2u * (4u * jp + 2u + h));
    }
    static __device__ __forceinline__ void partials(const W &w, const X &x, uint32_t, int32_t &a, int32_t &b) {
        int32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo = dot4(w.q[i] & 0x0F0F0F0Fu, x.lo[i], lo);
            hi = dot4((w.q[i] >> 4) & 0x0F0F0F0Fu, x.hi[i], hi);
        }
        a = w.sc1 * lo + w.sc2 * hi;
        b = w.m1 * x.bl + w.m2 * x.bh;
    }
    static __device__ __forceinline__ float term(const W &w, float d8, int32_t a, int32_t b) {
#pragma clang fp contract(off)
        const float dd = w.d * d8, dm = w.dmin * d8;
        return dd * (float)a - dm * (float)b;
    }
};

/* Q6_K (ql[128], qh[64], int8 scales[16], fp16 d; 210 bytes, so blocks are
 * only 2-byte aligned): part p = half p/4, columns l in 8(p%4)..+8 of the
 * half's four 32-groups; a = sum(sc*u*q8), b = sc[2p]*bsum[2p] +
 * sc[2p+1]*bsum[2p+1]; term = (d*d8) * (float)(a - 32*b)
 * (include/lfm2_simd_avx2.h:551-634). */
template <> struct QType<14> {
    static constexpr uint32_t kBytes = 210u;
    static constexpr bool kFloatParts = false;
    struct W { uint32_t l0[2], l1[2], qh[2]; int32_t s[4], so0, so1; float d; };
    struct X { float d8; uint32_t x[4][2]; int32_t b0, b1; };
    static __device__ __forceinline__ void load_w(W &w, const uint8_t *blk, uint32_t p) {
        const uint32_t half = p >> 2, q = p & 3u;
        const uint8_t *ql = blk + 64u * half + 8u * q, *qh = blk + 128u + 32u * half + 8u * q;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            w.l0[i] = ld16x2(ql + 4u * i);
            w.l1[i] = ld16x2(ql + 32u + 4u * i);
            w.qh[i] = ld16x2(qh + 4u * i);
        }
        const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192u + 8u * half + (q >> 1));
        w.s[0] = sc[0];
        w.s[1] = sc[2];
        w.s[2] = sc[4];
        w.s[3] = sc[6];
        const int8_t *so = reinterpret_cast<const int8_t *>(blk + 192u + 2u * p);
        w.so0 = so[0];
        w.so1 = so[1];
        w.d   = fp16_bits(*reinterpret_cast<const uint16_t *>(blk + 208u));
    }
    static __device__ __forceinline__ void load_x(X &x, const uint8_t *xb, uint32_t p) {
        const uint32_t half = p >> 2, q = p & 3u;
        x.d8 = *reinterpret_cast<const float *>(xb);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint8_t *g = xb + 4u + 128u * half + 32u * k + 8u * q;
            x.x[k][0] = ld32(g);
            x.x[k][1] = ld32(g + 4u);
        }
        const uint32_t bs = ld32(xb + 260u + 4u * p); /* bsums 2p, 2p+1 */
        x.b0 = (int16_t)(bs & 0xFFFFu);
        x.b1 = (int16_t)(bs >> 16);
    }
    static __device__ __forceinline__ void partials(const W &w, const X &x, uint32_t, int32_t &a, int32_t &b) {
        int32_t acc = 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t u1 = (w.l0[i] & 0x0F0F0F0Fu) | ((w.qh[i] & 0x03030303u) << 4);
            const uint32_t u2 = (w.l1[i] & 0x0F0F0F0Fu) | ((w.qh[i] & 0x0C0C0C0Cu) << 2);
            const uint32_t u3 = ((w.l0[i] >> 4) & 0x0F0F0F0Fu) | (w.qh[i] & 0x30303030u);
            const uint32_t u4 = ((w.l1[i] >> 4) & 0x0F0F0F0Fu) | ((w.qh[i] >> 2) & 0x30303030u);
            acc += w.s[0] * dot4(u1, x.x[0][i], 0) + w.s[1] * dot4(u2, x.x[1][i], 0) +
                   w.s[2] * dot4(u3, x.x[2][i], 0) + w.s[3] * dot4(u4, x.x[3][i], 0);
        }
        a = acc;
        b = w.so0 * x.b0 + w.so1 * x.b1;
    }
    static __device__ __forceinline__ float term(const W &w, float d8, int32_t a, int32_t b) {
#pragma clang fp contract(off)
        const float dd = w.d * d8;
        return dd * (float)(a - 32 * b);
    }
};

/* Q5_K (fp16 d, fp16 dmin, scales[12] as Q4_K, qh[32], qs[128]; 176 bytes):
 * part p = qs bytes 16p..16p+15 of 64-chunk c = p/2 with qh bytes
 * 16(p%2)..+15: low nibbles + 16 * qh bit 2c are sub-block 2c, high nibbles
 * + 16 * bit 2c+1 sub-block 2c+1; a, b and the term as Q4_K
 * (lfm2_vec_dot_q5_K_q8_K_avx2, tools/lfm2_cpuid_quants.c:690-740). */
template <> struct QType<13> {
    static constexpr uint32_t kBytes = 176u;
    static constexpr bool kFloatParts = false;
    using X = QType<12>::X;
    struct W { uint32_t lo[4], hi[4]; int32_t sc1, m1, sc2, m2; float d, dmin; };
    static __device__ __forceinline__ void load_w(W &w, const uint8_t *blk, uint32_t p) {
        const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qs  = *reinterpret_cast<const uint4 *>(blk + 48u + 16u * p);
        const uint4 qh  = *reinterpret_cast<const uint4 *>(blk + 16u + 16u * (p & 1u));
        const uint32_t c = p >> 1;
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w}, h[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w.lo[i] = (q[i] & 0x0F0F0F0Fu) | (((h[i] >> (2u * c)) & 0x01010101u) << 4);
            w.hi[i] = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (2u * c + 1u)) & 0x01010101u) << 4);
        }
        scale_min(2u * c, hdr.y, hdr.z, hdr.w, &w.sc1, &w.m1);
        scale_min(2u * c + 1u, hdr.y, hdr.z, hdr.w, &w.sc2, &w.m2);
        w.d    = fp16_bits(hdr.x & 0xFFFFu);
        w.dmin = fp16_bits(hdr.x >> 16);
    }
    static __device__ __forceinline__ void load_x(X &x, const uint8_t *xb, uint32_t p) { QType<12>::load_x(x, xb, p); }
    static __device__ __forceinline__ void partials(const W &w, const X &x, uint32_t, int32_t &a, int32_t &b) {
        int32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo = dot4(w.lo[i], x.lo[i], lo);
            hi = dot4(w.hi[i], x.hi[i], hi);
        }
        a = w.sc1 * lo + w.sc2 * hi;
        b = w.m1 * x.bl + w.m2 * x.bh;
    }
    static __device__ __forceinline__ float term(const W &w, float d8, int32_t a, int32_t b) {
#pragma clang fp contract(off)
        const float dd = w.d * d8, dm = w.dmin * d8;
        return dd * (float)a - dm * (float)b;
    }
};

/* IQ4_XS (fp16 d, scales_h, scales_l[4], qs[128]; 136 bytes): part p =
 * sub-block p, qs bytes 16p..16p+15 (low nibbles elements 0..15, high
 * 16..31) mapped through the IQ4_NL grid with v_perm_b32; a = ls * dot, b = 0;
 * term = (d*d8) * a (lfm2_vec_dot_iq4_xs_q8_K_avx2, tools/lfm2_cpuid_quants.c:832-880). */
template <> struct QType<23> {
    static constexpr uint32_t kBytes = 136u;
    static constexpr bool kFloatParts = false;
    struct W { uint32_t lo[4], hi[4]; int32_t ls; float d; };
    struct X { float d8; uint32_t lo[4], hi[4]; };
    /* the 16 grid values as int8 bytes, four per dword */
    static constexpr uint32_t kG0 = 0xBFAD9881u, kG1 = 0xF6EADDCFu, kG2 = 0x26190D01u, kG3 = 0x71594535u;
    static __device__ __forceinline__ uint32_t grid4(uint32_t nib) { /* 4 nibbles (one per byte) */
        const uint32_t sel = nib & 0x07070707u;
        const uint32_t lo  = __builtin_amdgcn_perm(kG1, kG0, sel);
        const uint32_t hi  = __builtin_amdgcn_perm(kG3, kG2, sel);
        const uint32_t m   = ((nib >> 3) & 0x01010101u) * 0xFFu;
        return (lo & ~m) | (hi & m);
    }
    static __device__ __forceinline__ void load_w(W &w, const uint8_t *blk, uint32_t p) {
        const uint2 hdr = *reinterpret_cast<const uint2 *>(blk);
        const uint2 q0  = *reinterpret_cast<const uint2 *>(blk + 8u + 16u * p);
        const uint2 q1  = *reinterpret_cast<const uint2 *>(blk + 16u + 16u * p);
        const uint32_t q[4] = {q0.x, q0.y, q1.x, q1.y};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w.lo[i] = grid4(q[i] & 0x0F0F0F0Fu);
            w.hi[i] = grid4((q[i] >> 4) & 0x0F0F0F0Fu);
        }
        const uint32_t sh = hdr.x >> 16, sl = hdr.y;
        w.ls = (int32_t)(((sl >> (8u * (p >> 1) + 4u * (p & 1u))) & 0x0Fu) | (((sh >> (2u * p)) & 3u) << 4)) - 32;
        w.d  = fp16_bits(hdr.x & 0xFFFFu);
    }
    static __device__ __forceinline__ void load_x(X &x, const uint8_t *xb, uint32_t p) {
        x.d8 = *reinterpret_cast<const float *>(xb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x.lo[i] = ld32(xb + 4u + 32u * p + 4u * i);
            x.hi[i] = ld32(xb + 20u + 32u * p + 4u * i);
        }
    }
    static __device__ __forceinline__ void partials(const W &w, const X &x, uint32_t, int32_t &a, int32_t &b) {
        int32_t acc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = dot4(w.hi[i], x.hi[i], dot4(w.lo[i], x.lo[i], acc));
        a = w.ls * acc;
        b = 0;
    }
    static __device__ __forceinline__ float term(const W &w, float d8, int32_t a, int32_t) {
#pragma clang fp contract(off)
        const float dd = w.d * d8;
        return dd * (float)a;
    }
};

/* Q4_0 (fp16 d, qs[16]; 18 bytes per 32 weights, 2-byte aligned): part p =
 * block p of the super-block; its float d * (sum(u4*q8) - 8 * bsums) is
 * summed in block order (lfm2_vec_dot_q4_0_q8_K_avx2,
 * tools/lfm2_cpuid_quants.c:634-672). */
template <> struct QType<2> {
    static constexpr uint32_t kBytes = 144u; /* 8 blocks */
    static constexpr bool kFloatParts = true;
    struct W { uint32_t q[4]; float d; };
    struct X { float d8; uint32_t lo[4], hi[4]; int32_t s8; };
    static __device__ __forceinline__ void load_w(W &w, const uint8_t *blk, uint32_t p) {
        const uint8_t *b = blk + 18u * p;
        w.d = fp16_bits(*reinterpret_cast<const uint16_t *>(b));
#pragma unroll
        for (int i = 0; i < 4; ++i) w.q[i] = ld16x2(b + 2u + 4u * i);
    }
    static __device__ __forceinline__ void load_x(X &x, const uint8_t *xb, uint32_t p) {
        x.d8 = *reinterpret_cast<const float *>(xb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x.lo[i] = ld32(xb + 4u + 32u * p + 4u * i);
            x.hi[i] = ld32(xb + 20u + 32u * p + 4u * i);
        }
        const uint32_t bs = ld32(xb + 260u + 4u * p);
        x.s8 = (int32_t)(int16_t)(bs & 0xFFFFu) + (int32_t)(int16_t)(bs >> 16);
    }
    static __device__ __forceinline__ float part_float(const W &w, const X &x) {
#pragma clang fp contract(off)
        int32_t acc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = dot4((w.q[i] >> 4) & 0x0F0F0F0Fu, x.hi[i], dot4(w.q[i] & 0x0F0F0F0Fu, x.lo[i], acc));
        return w.d * (float)(acc - 8 * x.s8);
    }
};

/* Q8_0 (fp16 d, int8 qs[32]; 34 bytes per 32 weights, 2-byte aligned): as
 * Q4_0 with d * sum(q*q8) (lfm2_vec_dot_q8_0_q8_K_avx2, include/lfm2_simd_avx2.h:639-674). */
template <> struct QType<8> {
    static constexpr uint32_t kBytes = 272u; /* 8 blocks */
    static constexpr bool kFloatParts = true;
    struct W { uint32_t q[8]; float d; };
    struct X { float d8; uint32_t v[8]; };
    static __device__ __forceinline__ void load_w(W &w, const uint8_t *blk, uint32_t p) {
        const uint8_t *b = blk + 34u * p;
        w.d = fp16_bits(*reinterpret_cast<const uint16_t *>(b));
#pragma unroll
        for (int i = 0; i < 8; ++i) w.q[i] = ld16x2(b + 2u + 4u * i);
    }
    static __device__ __forceinline__ void load_x(X &x, const uint8_t *xb, uint32_t p) {
        x.d8 = *reinterpret_cast<const float *>(xb);
#pragma unroll
        for (int i = 0; i < 8; ++i) x.v[i] = ld32(xb + 4u + 32u * p + 4u * i);
    }
    static __device__ __forceinline__ float part_float(const W &w, const X &x) {
#pragma clang fp contract(off)
        int32_t acc = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = dot4(w.q[i], x.v[i], acc);
        return w.d * (float)acc;
    }
};

/* Up to four matrices over the same activations (Q, K, V, gate), each of its
 * own GGML type; waves [wave0[m], wave0[m+1]) cover matrix m, RPW rows each. */
struct MatSet {
    const uint8_t *w[4];
    float *out[4];
    uint32_t rows[4];
    uint32_t type[4];
    uint32_t wave0[5];
    uint32_t n;
};

/* ---- quantized weights x Q8_K: out[t][r] ----------------------------------------
 * RPW rows of one matrix and a chunk of TCH tokens per wave (grid y = token
 * chunks): per 8-super-block step a lane loads its part of the RPW rows'
 * weights and of the TCH tokens' activations in one batch, then forms the
 * RPW x TCH partials, sums them over its lane group, and adds the
 * super-blocks' terms to the row sums in order. */
template <int TYPE, int RPW, int TCH>
__device__ __forceinline__ void matmul_rows(const uint8_t *__restrict__ w, float *__restrict__ out, uint32_t n_rows,
                                            uint32_t r0, const uint8_t *__restrict__ xq, uint32_t nb,
                                            uint32_t n_tokens, uint32_t t0) {
    using Q = QType<TYPE>;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t p = lane & 7u; /* part within the super-block    */
    const uint32_t g = lane >> 3; /* super-block slot of this step  */
    const size_t row_bytes = (size_t)nb * Q::kBytes;

    float sumf[TCH][RPW];
#pragma unroll
    for (int tt = 0; tt < TCH; ++tt)
#pragma unroll
        for (int r = 0; r < RPW; ++r) sumf[tt][r] = 0.0f;
    for (uint32_t b0 = 0; b0 < nb; b0 += 8u) {
        const uint32_t b = min(b0 + g, nb - 1u); /* slots past the end repeat a block, unused */
        typename Q::W wr[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint32_t row = min(r0 + (uint32_t)r, n_rows - 1u);
            Q::load_w(wr[r], w + row * row_bytes + (size_t)b * Q::kBytes, p);
        }
        typename Q::X xt[TCH];
#pragma unroll
        for (int tt = 0; tt < TCH; ++tt) {
            const uint32_t t = min(t0 + (uint32_t)tt, n_tokens - 1u);
            Q::load_x(xt[tt], xq + ((size_t)t * nb + b) * kQ8K, p);
        }
        float term[TCH][RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int tt = 0; tt < TCH; ++tt) {
                if constexpr (Q::kFloatParts) {
                    /* blocks of the super-block in order, then times d8 */
                    const float t  = Q::part_float(wr[r], xt[tt]);
                    const int base = (int)(lane & ~7u);
                    float bsum     = add_rounded(0.0f, __shfl(t, base));
#pragma unroll
                    for (int k = 1; k < 8; ++k) bsum = add_rounded(bsum, __shfl(t, base + k));
                    term[tt][r] = mul_rounded(xt[tt].d8, bsum);
                } else {
                    int32_t a, c;
                    Q::partials(wr[r], xt[tt], p, a, c);
#pragma unroll
                    for (int o = 1; o < 8; o <<= 1) {
                        a += __shfl_xor(a, o);
                        c += __shfl_xor(c, o);
                    }
                    term[tt][r] = Q::term(wr[r], xt[tt].d8, a, c);
                }
            }
        /* super-blocks b0 .. b0+7 in order; a block whose d8 is 0 adds nothing */
#pragma unroll
        for (uint32_t i = 0; i < 8u; ++i) {
            if (b0 + i >= nb) break;
#pragma unroll
            for (int tt = 0; tt < TCH; ++tt) {
                const float d8i = __shfl(xt[tt].d8, (int)(8u * i));
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const float ti = __shfl(term[tt][r], (int)(8u * i));
                    if (d8i != 0.0f) sumf[tt][r] = add_rounded(sumf[tt][r], ti);
                }
            }
        }
    }
    /* lane tt * RPW + r writes token t0 + tt, row r0 + r */
#pragma unroll
    for (int tt = 0; tt < TCH; ++tt)
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            if (lane == (uint32_t)(tt * RPW + r) && t0 + tt < n_tokens && r0 + r < n_rows)
                out[(size_t)(t0 + tt) * n_rows + r0 + r] = sumf[tt][r];
}

/* one launch over every matrix of the set.  TYPE > 0: all matrices of that
 * type; TYPE == 0: each wave takes its matrix's type (a wave-uniform branch;
 * the kernel then needs the registers of the widest type, so sets of one
 * type take the specialised form) */
template <int TYPE, int RPW, int TCH>
__global__ __launch_bounds__(256) void k_matmul_q(const MatSet S, const uint8_t *__restrict__ xq, uint32_t nb,
                                                  uint32_t n_tokens) {
    const uint32_t wv = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (wv >= S.wave0[S.n]) return;
    uint32_t m = 0;
    while (m + 1u < S.n && wv >= S.wave0[m + 1u]) ++m;
    const uint32_t r0 = (wv - S.wave0[m]) * RPW, t0 = blockIdx.y * TCH;
    if constexpr (TYPE != 0) {
        matmul_rows<TYPE, RPW, TCH>(S.w[m], S.out[m], S.rows[m], r0, xq, nb, n_tokens, t0);
        return;
    }
    switch (S.type[m]) {
    case 12u: matmul_rows<12, RPW, TCH>(S.w[m], S.out[m], S.rows[m], r0, xq, nb, n_tokens, t0); break;
    case 14u: matmul_rows<14, RPW, TCH>(S.w[m], S.out[m], S.rows[m], r0, xq, nb, n_tokens, t0); break;
    case 13u: matmul_rows<13, RPW, TCH>(S.w[m], S.out[m], S.rows[m], r0, xq, nb, n_tokens, t0); break;
    case 23u: matmul_rows<23, RPW, TCH>(S.w[m], S.out[m], S.rows[m], r0, xq, nb, n_tokens, t0); break;
    case 2u: matmul_rows<2, RPW, TCH>(S.w[m], S.out[m], S.rows[m], r0, xq, nb, n_tokens, t0); break;
    default: matmul_rows<8, RPW, TCH>(S.w[m], S.out[m], S.rows[m], r0, xq, nb, n_tokens, t0); break;
    }
}

template <int TYPE, int RPW, int TCH>
hipError_t launch_set(MatSet S, const void *x_q8, uint32_t nb, uint32_t n_tokens, hipStream_t stream) {
    S.wave0[0] = 0;
    for (uint32_t m = 0; m < S.n; ++m) S.wave0[m + 1] = S.wave0[m] + (S.rows[m] + RPW - 1u) / RPW;
    if (S.wave0[S.n] == 0u) return hipSuccess;
    hipLaunchKernelGGL((k_matmul_q<TYPE, RPW, TCH>), dim3((S.wave0[S.n] + 3u) / 4u, (n_tokens + TCH - 1u) / TCH),
                       dim3(256), 0, stream, S, static_cast<const uint8_t *>(x_q8), nb, n_tokens);
    return hipGetLastError();
}

/* one token: a row per wave (most waves in flight); more: two rows and up to
 * eight tokens per wave share each weight and activation load */
template <int TYPE>
hipError_t launch_tokens(const MatSet &S, const void *x_q8, uint32_t nb, uint32_t n_tokens, hipStream_t stream) {
    if (n_tokens == 1u) return launch_set<TYPE, 1, 1>(S, x_q8, nb, n_tokens, stream);
    if (n_tokens == 2u) return launch_set<TYPE, 2, 2>(S, x_q8, nb, n_tokens, stream);
    if (n_tokens <= 4u) return launch_set<TYPE, 2, 4>(S, x_q8, nb, n_tokens, stream);
    return launch_set<TYPE, 2, 8>(S, x_q8, nb, n_tokens, stream);
}

/* ---- Q4_K / Q5_K x Q8_K on int8 MFMA, 8 or more tokens -------------------------
 * A workgroup computes a 16-token x 16-row tile with the reference's exact
 * integer sums and its fp32 rounding order.  Per super-block:
 *   per sub-block j   dot_j[t][r] = sum_32 q8[t] * q4[r]  v_mfma_i32_16x16x32_i8
 *                     (A = the tokens' int8 activations, B = the row's 4-bit
 *                     weights, with Q5_K's fifth bit from qh ORed in)
 *   a[t][r] = sum_j sc_j[r] * dot_j[t][r]                 int32 on the VALU
 *   b[t][r] = sum_j m_j[r] * (bsum[t][2j] + bsum[t][2j+1])  two
 *             v_mfma_f32_16x16x4_f32 on integers below 2^24, hence exact
 *   term[t][r] = (d*d8)*a - (dmin*d8)*b  every product and sum rounded
 * The four waves compute the terms of different super-blocks (a term depends
 * on its super-block alone); then each thread adds its element's terms in
 * super-block order, a super-block whose d8 is 0 adding nothing, so the result
 * is bit-identical to the one-token-at-a-time kernel.  Lane (l16, g) of a wave
 * supplies token t0 + l16 (A) and row r0 + l16 (B) over k-slice g, and holds
 * the terms of tokens t0 + 4g + i, row r0 + l16. */
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float sub_rounded(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

__device__ __forceinline__ long ld64_4(const uint8_t *p) { /* 4-byte aligned */
    return (long)(((uint64_t)ld32(p + 4) << 32) | ld32(p));
}

constexpr uint32_t kMfmaChunk = 8u; /* super-blocks per round (two per wave) */

template <int TYPE>
__global__ __launch_bounds__(256) void k_matmul_qk_mfma(const uint8_t *__restrict__ w, float *__restrict__ out,
                                                        uint32_t n_rows, const uint8_t *__restrict__ xq,
                                                        uint32_t nb, uint32_t n_tokens) {
    static_assert(TYPE == 12 || TYPE == 13, "Q4_K or Q5_K");
    constexpr uint32_t kBytes = QType<TYPE>::kBytes, kQs = TYPE == 12 ? 16u : 48u;
    __shared__ float terms[kMfmaChunk][256];   /* [super-block of the round][token * 16 + row] */
    __shared__ uint32_t live[kMfmaChunk][16];  /* d8 != 0 per [super-block][token] */
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, l16 = lane & 15u, g = lane >> 4;
    const uint32_t r0 = blockIdx.x * 16u, t0 = blockIdx.y * 16u;
    const uint8_t *wr = w + (size_t)(r0 + l16) * nb * kBytes;
    const uint8_t *xa = xq + (size_t)min(t0 + l16, n_tokens - 1u) * nb * kQ8K;
    const uint8_t *xd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xd[i] = xq + (size_t)min(t0 + 4u * g + (uint32_t)i, n_tokens - 1u) * nb * kQ8K;
    float sumf = 0.0f; /* element tid: token t0 + tid / 16, row r0 + tid % 16 */
    for (uint32_t c0 = 0; c0 < nb; c0 += kMfmaChunk) {
#pragma unroll
        for (uint32_t u = 0; u < 2u; ++u) {
            const uint32_t k = 2u * wave + u, b = c0 + k;
            if (b >= nb) break;
            const uint8_t *blk = wr + (size_t)b * kBytes;
            const uint8_t *xb  = xa + (size_t)b * kQ8K;
            const uint4 hdr    = *reinterpret_cast<const uint4 *>(blk);
            int32_t sc[8], mn_unused, m_lo, m_hi, sc_unused;
#pragma unroll
            for (uint32_t j = 0; j < 8u; ++j) scale_min(j, hdr.y, hdr.z, hdr.w, &sc[j], &mn_unused);
            /* mins of sub-blocks g and g + 4: this lane's k-slice of the mins product */
            scale_min(g, hdr.y, hdr.z, hdr.w, &sc_unused, &m_lo);
            scale_min(g + 4u, hdr.y, hdr.z, hdr.w, &sc_unused, &m_hi);
            i32x4_t a = (i32x4_t)0;
            uint2 qh = make_uint2(0u, 0u); /* Q5_K: bit j of qh[i] is weight i's fifth bit in sub-block j */
            if constexpr (TYPE == 13) qh = *reinterpret_cast<const uint2 *>(blk + 16u + 8u * g);
#pragma unroll
            for (uint32_t jp = 0; jp < 4u; ++jp) {
                const uint2 wq = *reinterpret_cast<const uint2 *>(blk + kQs + 32u * jp + 8u * g);
                uint32_t lx = wq.x & 0x0F0F0F0Fu, ly = wq.y & 0x0F0F0F0Fu;
                uint32_t hx = (wq.x >> 4) & 0x0F0F0F0Fu, hy = (wq.y >> 4) & 0x0F0F0F0Fu;
                if constexpr (TYPE == 13) {
                    lx |= ((qh.x >> (2u * jp)) & 0x01010101u) << 4;
                    ly |= ((qh.y >> (2u * jp)) & 0x01010101u) << 4;
                    hx |= ((qh.x >> (2u * jp + 1u)) & 0x01010101u) << 4;
                    hy |= ((qh.y >> (2u * jp + 1u)) & 0x01010101u) << 4;
                }
                const long blo = (long)(((uint64_t)ly << 32) | lx);
                const long bhi = (long)(((uint64_t)hy << 32) | hx);
                const long alo = ld64_4(xb + 4u + 32u * (2u * jp) + 8u * g);
                const long ahi = ld64_4(xb + 4u + 32u * (2u * jp + 1u) + 8u * g);
                const i32x4_t dlo = __builtin_amdgcn_mfma_i32_16x16x32_i8(alo, blo, (i32x4_t)0, 0, 0, 0);
                const i32x4_t dhi = __builtin_amdgcn_mfma_i32_16x16x32_i8(ahi, bhi, (i32x4_t)0, 0, 0, 0);
                a += sc[2u * jp] * dlo + sc[2u * jp + 1u] * dhi;
            }
            const uint32_t p0 = ld32(xb + 260u + 4u * g), p1 = ld32(xb + 260u + 4u * (g + 4u));
            const float bs0 = (float)((int32_t)(int16_t)(p0 & 0xFFFFu) + (int32_t)(int16_t)(p0 >> 16));
            const float bs1 = (float)((int32_t)(int16_t)(p1 & 0xFFFFu) + (int32_t)(int16_t)(p1 >> 16));
            f32x4_t bm = __builtin_amdgcn_mfma_f32_16x16x4f32(bs0, (float)m_lo, (f32x4_t)0.0f, 0, 0, 0);
            bm         = __builtin_amdgcn_mfma_f32_16x16x4f32(bs1, (float)m_hi, bm, 0, 0, 0);
            const float d = fp16_bits(hdr.x & 0xFFFFu), dmin = fp16_bits(hdr.x >> 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float d8 = *reinterpret_cast<const float *>(xd[i] + (size_t)b * kQ8K);
                terms[k][(4u * g + (uint32_t)i) * 16u + l16] =
                    sub_rounded(mul_rounded(mul_rounded(d, d8), (float)a[i]), mul_rounded(mul_rounded(dmin, d8), bm[i]));
            }
            if (g == 0u) live[k][l16] = *reinterpret_cast<const float *>(xb) != 0.0f;
        }
        __syncthreads();
        const uint32_t n_k = min(kMfmaChunk, nb - c0);
        for (uint32_t k = 0; k < n_k; ++k)
            if (live[k][tid >> 4]) sumf = add_rounded(sumf, terms[k][tid]);
        __syncthreads();
    }
    const uint32_t t = t0 + (tid >> 4);
    if (t < n_tokens) out[(size_t)t * n_rows + r0 + (tid & 15u)] = sumf;
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

int launch_matmul_q(uint32_t n_mats, float *const *outs, const void *const *ws, const uint32_t *types,
                    const uint32_t *rows, uint32_t n_cols, const void *x_q8, uint32_t n_tokens, hipStream_t stream) {
    if (n_tokens == 0u) return LFM_ATTN_OK;
    const uint32_t nb = n_cols / 256u;
    /* one launch over all matrices, whatever their types */
    MatSet S{};
    for (uint32_t m = 0; m < n_mats && m < 4u; ++m) {
        if (rows[m] == 0u) continue;
        S.w[S.n]    = static_cast<const uint8_t *>(ws[m]);
        S.out[S.n]  = outs[m];
        S.rows[S.n] = rows[m];
        S.type[S.n] = types[m];
        ++S.n;
    }
    if (S.n == 0u) return LFM_ATTN_OK;
    bool one_type = true;
    for (uint32_t m = 1; m < S.n; ++m) one_type = one_type && S.type[m] == S.type[0];
    hipError_t e;
    /* >= 8 tokens: each Q4_K or Q5_K matrix of whole 16-row tiles goes to the
     * int8-MFMA kernel (measured on MI355X, Q4_K 2048 x 2048: 8 tokens
     * 8.8 -> 6.3 us, 64 tokens 36 -> 8.8 us against the dot4 path); the
     * other matrices of the set stay in one dot4 launch */
    if (n_tokens >= 8u) {
        MatSet R{};
        const uint8_t *xq = static_cast<const uint8_t *>(x_q8);
        for (uint32_t m = 0; m < S.n; ++m) {
            const bool mfma = (S.type[m] == 12u || S.type[m] == 13u) && S.rows[m] % 16u == 0u;
            if (!mfma) {
                R.w[R.n] = S.w[m];
                R.out[R.n] = S.out[m];
                R.rows[R.n] = S.rows[m];
                R.type[R.n] = S.type[m];
                ++R.n;
                continue;
            }
            const dim3 grid(S.rows[m] / 16u, (n_tokens + 15u) / 16u);
            if (S.type[m] == 12u)
                hipLaunchKernelGGL(k_matmul_qk_mfma<12>, grid, dim3(256), 0, stream, S.w[m], S.out[m], S.rows[m], xq,
                                   nb, n_tokens);
            else
                hipLaunchKernelGGL(k_matmul_qk_mfma<13>, grid, dim3(256), 0, stream, S.w[m], S.out[m], S.rows[m], xq,
                                   nb, n_tokens);
            const hipError_t le = hipGetLastError();
            if (le != hipSuccess) return hip_status(le);
        }
        if (R.n == 0u) return LFM_ATTN_OK;
        S = R;
        one_type = true;
        for (uint32_t m = 1; m < S.n; ++m) one_type = one_type && S.type[m] == S.type[0];
    }
    switch (one_type ? S.type[0] : 0u) {
    case 12u: e = launch_tokens<12>(S, x_q8, nb, n_tokens, stream); break;
    case 14u: e = launch_tokens<14>(S, x_q8, nb, n_tokens, stream); break;
    case 13u: e = launch_tokens<13>(S, x_q8, nb, n_tokens, stream); break;
    case 23u: e = launch_tokens<23>(S, x_q8, nb, n_tokens, stream); break;
    case 2u: e = launch_tokens<2>(S, x_q8, nb, n_tokens, stream); break;
    case 8u: e = launch_tokens<8>(S, x_q8, nb, n_tokens, stream); break;
    default: e = launch_tokens<0>(S, x_q8, nb, n_tokens, stream); break;
    }
    return hip_status(e);
}

} // namespace lfm
