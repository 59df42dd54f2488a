/*
 * prefill_fa.hip -- causal prefill attention on gfx950 MFMA (fp16 Q/K/V,
 * fp32 softmax and accumulation, fp32 output).
 *
 * Semantics: lfm2_forward_gqa_batch (tools/lfm2_prefill_batch.c:1029-1092)
 * runs the per-head task once per query row; row i (position pos_0 + i)
 * attends keys [0, pos_0 + i] of its cache (causal by write order).  This
 * kernel computes all rows of a prompt in one launch.
 *
 * Workgroup = 4 waves = TQ query positions x kv_mul query heads of one KV
 * head (256 query columns, TQ = 256 / kv_mul), so each K/V block staged in
 * LDS serves every query head that reads it.  Per 64-key block:
 *   S^T = K . Q^T - m    16x16x32 f16 MFMA; K fragments from LDS, Q^T from
 *                        registers; the running max enters as the
 *                        accumulator's initial value (no per-score subtract).
 *   p = exp2(S^T)        lazy max: the running max is raised only when a
 *                        block exceeds it by more than 2^8 (fp16 P stays
 *                        finite), which rescales O and l.
 *   l += p               v_dot2_f32_f16 over the fp16 P actually fed to the
 *                        MFMA, so numerator and denominator use the same P.
 *   O^T += V^T . P^T     V^T fragments from LDS (V is transposed while it is
 *                        staged), P^T straight from the S^T accumulator layout.
 * Causal masking only touches blocks that cross the diagonal; blocks above it
 * are skipped.  Workgroups run heaviest-first (late query tiles first).
 */
#include <hip/hip_runtime.h>

#include <type_traits>

#include "kernels.h"
#include "lfm_attn.h"

namespace lfm {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int KB       = 64;      /* keys per block                         */
constexpr int KSTR     = 64 + 8;  /* halfs per K row in LDS (16 B pad)      */
constexpr int VSTR     = KB + 8;  /* halfs per d row of V^T in LDS (16 B pad) */
constexpr float kLazy  = 8.0f;    /* log2 headroom before the max is raised */

struct PrefillParams {
    const uint16_t *q;  /* [n_seq][n_tok][n_head_q][HD] fp16 */
    const uint16_t *k;  /* seq s at k + s*kv_seq_stride: [slot][n_head_kv][HD] */
    const uint16_t *v;
    float *out;         /* [n_seq][n_tok][n_head_q][HD] */
    uint64_t kv_seq_stride;
    uint32_t n_seq, n_tok, pos_0, n_head_q, n_head_kv, kv_mul, tq, n_qtiles;
    float qscale;       /* scale * log2(e) */
};

__device__ __forceinline__ half8_t as_half8(u32x4_t v) { return __builtin_bit_cast(half8_t, v); }

__device__ __forceinline__ float4_t mfma(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

/* exp2 of two scores packed to fp16 (round toward zero) */
__device__ __forceinline__ half2_t exp2_pk(float a, float b) {
    return __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(__builtin_amdgcn_exp2f(a),
                                                                  __builtin_amdgcn_exp2f(b)));
}

template <int HD>
__global__ __launch_bounds__(256, 2) void k_prefill(const PrefillParams P) {
    static_assert(HD == 64, "prefill kernel is specialised for head_dim 64");
    constexpr int NT = 4; /* 16-column tiles per wave (64 columns)         */
    constexpr int MT = 4; /* 16-key tiles per block                        */
    constexpr int NM = HD / 16;
    __shared__ __attribute__((aligned(16))) uint16_t ks[2][KB * KSTR];
    __shared__ __attribute__((aligned(16))) uint16_t vts[2][HD * VSTR];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    /* 1-D grid, heaviest query tiles first across all (sequence, KV head)
     * pairs; consecutive workgroups take consecutive pairs, so the tiles of
     * one pair all land on the same XCD (round-robin over 8) and share its L2 */
    const uint32_t pairs = P.n_head_kv * P.n_seq;
    const uint32_t qt    = P.n_qtiles - 1u - blockIdx.x / pairs;
    const uint32_t pair  = blockIdx.x % pairs;
    const uint32_t kvh = pair % P.n_head_kv, s = pair / P.n_head_kv;
    const uint32_t t0  = qt * P.tq; /* first query row of the tile */

    const uint16_t *kc = P.k + (size_t)s * P.kv_seq_stride + (size_t)kvh * HD;
    const uint16_t *vc = P.v + (size_t)s * P.kv_seq_stride + (size_t)kvh * HD;
    const size_t row   = (size_t)P.n_head_kv * HD;

    /* ---- columns of this lane: (head j, row t) per N-tile -------------- */
    uint32_t col_pos[NT]; /* absolute position of the column's query row */
    bool col_ok[NT];
    half8_t qf[NT][HD / 32];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t c = (uint32_t)(wave * 64 + nt * 16 + l16);
        const uint32_t j = c / P.tq, t = t0 + c % P.tq;
        col_ok[nt]  = t < P.n_tok;
        col_pos[nt] = P.pos_0 + t;
        const uint16_t *qp = P.q + (((size_t)s * P.n_tok + (col_ok[nt] ? t : 0u)) * P.n_head_q +
                                    kvh * P.kv_mul + j) * HD + 8 * g;
#pragma unroll
        for (int st = 0; st < HD / 32; ++st) {
            u32x4_t raw = col_ok[nt] ? *reinterpret_cast<const u32x4_t *>(qp + 32 * st) : (u32x4_t)0u;
            half8_t h   = as_half8(raw);
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (_Float16)((float)h[e] * P.qscale);
            qf[nt][st] = h;
        }
    }
    /* q*scale*log2(e) is rounded to fp16 once (relative error <= 2^-11 per
     * element), which keeps the score accumulator in log2 units */
    const uint32_t lo_pos = P.pos_0 + t0;                                   /* smallest query position */
    const uint32_t hi_pos = P.pos_0 + min(t0 + P.tq, P.n_tok) - 1u;         /* largest query position  */
    const uint32_t n_keys = hi_pos + 1u;
    const uint32_t nblk   = (n_keys + KB - 1) / KB;

    /* ---- staging: waves 0-1 load K rows, waves 2-3 load V (4 keys / lane) --
     * V^T is stored per d-row with the keys of each 32-key step permuted to
     * [0-3,16-19, 4-7,20-23, 8-11,24-27, 12-15,28-31], so the P^T-matching
     * A fragment of a lane (keys 4g..4g+3 and 16+4g..19+4g) is 16 contiguous
     * bytes: one ds_read_b128. */
    const int sc = tid & 7, srow = (tid & 127) >> 3;
    const uint16_t *sbase = (tid < 128 ? kc + (size_t)srow * row : vc + (size_t)(4 * srow) * row) + 8 * sc;
    const size_t sstep = (tid < 128 ? 16u : 1u) * row; /* between the 4 rows a lane loads */
    u32x4_t stage[4];
    auto load_block = [&](uint32_t kb) {
        const uint16_t *src = sbase + (size_t)kb * row;
        if (kb + KB <= n_keys) {
#pragma unroll
            for (int i = 0; i < 4; ++i) stage[i] = *reinterpret_cast<const u32x4_t *>(src + i * sstep);
        } else { /* last block: rows past the keys repeat the last key (masked) */
            const uint32_t r0 = tid < 128 ? (uint32_t)srow : 4u * srow;
            const uint32_t dr = tid < 128 ? 16u : 1u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t key = kb + r0 + dr * (uint32_t)i;
                key = key < n_keys ? key : n_keys - 1u;
                stage[i] = *reinterpret_cast<const u32x4_t *>((tid < 128 ? kc : vc) + (size_t)key * row + 8 * sc);
            }
        }
    };
    auto store_block = [&](int buf) {
        if (tid < 128) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<u32x4_t *>(&ks[buf][(srow + 16 * i) * KSTR + 8 * sc]) = stage[i];
        } else {
            const int quad = srow, j = quad >> 3, qq = quad & 7;
            const int pos  = 32 * j + 8 * (qq & 3) + 4 * (qq >> 2);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t a0 = stage[0][w], a1 = stage[1][w], a2 = stage[2][w], a3 = stage[3][w];
                u32x2_t even, odd;
                even[0] = (a0 & 0xFFFFu) | (a1 << 16);
                even[1] = (a2 & 0xFFFFu) | (a3 << 16);
                odd[0]  = (a0 >> 16) | (a1 & 0xFFFF0000u);
                odd[1]  = (a2 >> 16) | (a3 & 0xFFFF0000u);
                *reinterpret_cast<u32x2_t *>(&vts[buf][(8 * sc + 2 * w) * VSTR + pos])     = even;
                *reinterpret_cast<u32x2_t *>(&vts[buf][(8 * sc + 2 * w + 1) * VSTR + pos]) = odd;
            }
        }
    };

    float4_t oacc[NM][NT];
    float m[NT], l[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        m[nt] = 0.0f;
        l[nt] = 0.0f;
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] = (float4_t)0.0f;
    }
    const half2_t ones = {(_Float16)1.0f, (_Float16)1.0f};

    /* one 64-key block; MASK only on blocks crossing the lowest query row */
    auto block = [&](auto mask_tag, uint32_t b) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int buf     = (int)(b & 1u);
        const uint32_t kb = b * KB;
        float4_t sacc[MT][NT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const uint16_t *kr = &ks[buf][(16 * mt + l16) * KSTR + 8 * g];
            const half8_t k0 = as_half8(*reinterpret_cast<const u32x4_t *>(kr));
            const half8_t k1 = as_half8(*reinterpret_cast<const u32x4_t *>(kr + 32));
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                float4_t acc = (float4_t)(-m[nt]);
                acc = mfma(k0, qf[nt][0], acc);
                acc = mfma(k1, qf[nt][1], acc);
                sacc[mt][nt] = acc;
            }
        }
        if constexpr (MASK) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t key = kb + (uint32_t)(16 * mt + 4 * g + i);
                        if (key > col_pos[nt]) sacc[mt][nt][i] = -INFINITY;
                    }
        }
        /* block max relative to m: the first block sets m, later ones raise it
         * only past 2^kLazy (rare), in a wave-uniform branch */
        float mx[NT];
        bool any_raise = false;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float v = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                v = fmaxf(v, fmaxf(fmaxf(sacc[mt][nt][0], sacc[mt][nt][1]),
                                   fmaxf(sacc[mt][nt][2], sacc[mt][nt][3])));
            mx[nt] = v;
            any_raise |= (b == 0u) ? true : (v > kLazy);
        }
        if (__builtin_amdgcn_ballot_w64(any_raise) != 0ull) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                float v = mx[nt]; /* column max over the 4 lanes holding it */
                v = fmaxf(v, __shfl_xor(v, 16));
                v = fmaxf(v, __shfl_xor(v, 32));
                const bool raise  = (b == 0u) ? (v > -INFINITY) : (v > kLazy);
                const float inc   = raise ? v : 0.0f;
                const float alpha = __builtin_amdgcn_exp2f(-inc);
                m[nt] += inc;
                l[nt] *= alpha;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) sacc[mt][nt] -= inc;
#pragma unroll
                for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] *= alpha;
            }
        }
        /* per 32-key step: P^T fragments (fp16, RTZ), l from the same fp16
         * values, then O^T += V^T . P^T */
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            u32x4_t pf[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const float4_t a = sacc[2 * j][nt], c = sacc[2 * j + 1][nt];
                /* scalar temporaries: a bit_cast of an ext-vector element was
                 * miscompiled into four reads of element 0 */
                const half2_t h0 = exp2_pk(a[0], a[1]);
                const half2_t h1 = exp2_pk(a[2], a[3]);
                const half2_t h2 = exp2_pk(c[0], c[1]);
                const half2_t h3 = exp2_pk(c[2], c[3]);
                float lsum = l[nt];
                lsum = __builtin_amdgcn_fdot2(h0, ones, lsum, false);
                lsum = __builtin_amdgcn_fdot2(h1, ones, lsum, false);
                lsum = __builtin_amdgcn_fdot2(h2, ones, lsum, false);
                lsum = __builtin_amdgcn_fdot2(h3, ones, lsum, false);
                l[nt] = lsum;
                u32x4_t w;
                w[0] = __builtin_bit_cast(uint32_t, h0);
                w[1] = __builtin_bit_cast(uint32_t, h1);
                w[2] = __builtin_bit_cast(uint32_t, h2);
                w[3] = __builtin_bit_cast(uint32_t, h3);
                pf[nt] = w;
            }
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const half8_t av = as_half8(*reinterpret_cast<const u32x4_t *>(
                    &vts[buf][(16 * mt + l16) * VSTR + 32 * j + 8 * g]));
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) oacc[mt][nt] = mfma(av, as_half8(pf[nt]), oacc[mt][nt]);
            }
        }
    };

    /* blocks [0, nfull) lie entirely at or below the lowest query row */
    const uint32_t nfull = (lo_pos + 1u) / KB < nblk ? (lo_pos + 1u) / KB : nblk;
    load_block(0);
    store_block(0);
    __syncthreads();
    uint32_t b = 0;
    for (; b < nfull; ++b) {
        if (b + 1 < nblk) load_block((b + 1) * KB);
        block(std::integral_constant<bool, false>{}, b);
        if (b + 1 < nblk) store_block((int)((b + 1) & 1u));
        __syncthreads();
    }
    for (; b < nblk; ++b) {
        if (b + 1 < nblk) load_block((b + 1) * KB);
        block(std::integral_constant<bool, true>{}, b);
        if (b + 1 < nblk) store_block((int)((b + 1) & 1u));
        __syncthreads();
    }

    /* ---- epilogue: O / l ------------------------------------------------- */
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        float lt = l[nt] + __shfl_xor(l[nt], 16);
        lt += __shfl_xor(lt, 32);
        if (!col_ok[nt]) continue;
        const uint32_t c = (uint32_t)(wave * 64 + nt * 16 + l16);
        const uint32_t j = c / P.tq, t = t0 + c % P.tq;
        const float inv  = lt > 0.0f ? 1.0f / lt : 0.0f;
        float *op = P.out + (((size_t)s * P.n_tok + t) * P.n_head_q + kvh * P.kv_mul + j) * HD;
#pragma unroll
        for (int mt = 0; mt < NM; ++mt)
            *reinterpret_cast<float4 *>(op + 16 * mt + 4 * g) =
                make_float4(oacc[mt][nt][0] * inv, oacc[mt][nt][1] * inv, oacc[mt][nt][2] * inv,
                            oacc[mt][nt][3] * inv);
    }
}

} // namespace

bool prefill_supports(uint32_t head_dim, uint32_t kv_mul) {
    return head_dim == 64u && kv_mul >= 1u && kv_mul <= 16u && (256u % kv_mul) == 0u;
}

int launch_prefill(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *out,
                   uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint64_t kv_seq_stride,
                   uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim, float scale,
                   hipStream_t stream) {
    PrefillParams P{};
    P.q = q;
    P.k = k;
    P.v = v;
    P.out = out;
    P.kv_seq_stride = kv_seq_stride;
    P.n_seq = n_seq;
    P.n_tok = n_tok;
    P.pos_0 = pos_0;
    P.n_head_q = n_head_q;
    P.n_head_kv = n_head_kv;
    P.kv_mul = n_head_q / n_head_kv;
    P.tq = 256u / P.kv_mul;
    P.n_qtiles = (n_tok + P.tq - 1u) / P.tq;
    P.qscale = scale * kLog2e;
    hipEvent_t ev0, ev1;
    profile_events(&ev0, &ev1);
    if (ev0) (void)hipEventRecord(ev0, stream);
    hipLaunchKernelGGL(k_prefill<64>, dim3(P.n_qtiles * n_head_kv * n_seq), dim3(256), 0, stream, P);
    hipError_t e = hipGetLastError();
    if (ev1) (void)hipEventRecord(ev1, stream);
    (void)head_dim;
    return hip_status(e);
}

} // namespace lfm
