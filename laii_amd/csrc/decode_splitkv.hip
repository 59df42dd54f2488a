/*
 * decode_splitkv.hip -- split-KV online-softmax GQA attention over fp16 KV
 * caches on gfx950 MFMA (decode, B<=8 speculative verify, LFM3 SWA ring and
 * full layers).
 *
 * Reference semantics: tools/lfm2_kernels_fast.c:700-810 (A1),
 * tools/lfm2_threadpool.c:764-828 (A2 fp16 branch), tools/lfm3_engine.c:851-946
 * (A3: ring segments, gate epilogue o * gate / l).  The softmax is the same
 * mathematical function; keys are visited in 32-key sub-tiles instead of one
 * at a time, and partial results of key splits are merged by log-sum-exp.
 *
 * Work decomposition: one wave64 workgroup per (key split, KV head, sequence).
 * The wave owns every query column that reads its KV head: column
 * n = row * kv_mul + j (row of the speculative batch, q head kvh*kv_mul + j),
 * so each K/V byte of the split is read from HBM exactly once.
 *
 * Per 32-key sub-tile:
 *   S^T[key][col] = K . Q^T      v_mfma_f32_16x16x32_f16, A = K rows loaded
 *                                straight from HBM (16 B per lane), B = Q^T.
 *                                Q is held as fp16 hi + lo (q*scale*log2e =
 *                                hi + lo), both accumulated into one S^T, so
 *                                scores keep ~fp32 accuracy.
 *   online softmax (exp2 domain) on the S^T accumulator: column max over the
 *                                8 scores a lane holds + 2 cross-row shuffles.
 *   O^T[d][col] += V^T . P^T     the S^T accumulator layout IS the B-operand
 *                                layout of the next MFMA (keys 4g..4g+3 and
 *                                16+4g..19+4g of column l%16), so P needs no
 *                                shuffle; P is split hi + lo like Q.  V^T comes
 *                                from LDS: V rows are loaded 16 B per lane,
 *                                stored row-major (XOR-swizzled 16-B chunks)
 *                                and read back transposed by
 *                                ds_read_b64_tr_b16.
 * Loads of sub-tile i+1 are issued before sub-tile i is consumed.
 */
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "attn_index.h"
#include "kernels.h"
#include "splitkv_plan.h"
#include "lfm_attn.h"

namespace lfm {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4v_t __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4;

/* transposing LDS read: within each 16-lane group, lane l receives element
 * l % 4 of the 8-byte chunks addressed by lanes l/4, l/4 + 4, l/4 + 8 and
 * l/4 + 12 */
__device__ __forceinline__ half4v_t lds_read_tr(const uint8_t *p) {
    return __builtin_bit_cast(half4v_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4 *)p));
}

constexpr float kLog2e     = 1.4426950408889634f;
constexpr float kNegBig    = -1e30f; /* running-max sentinel (finite)          */
constexpr float kLazyMax   = 8.0f;   /* running max raised only past m + 8 (log2 units) */
/* halfs of a wave's LDS V tile: 32 keys x head_dim, row-major */
template <int HD> constexpr int vt_halfs() { return 32 * HD; }

struct SplitParams {
    const float *q;
    const float *gate;
    const uint16_t *k_base;
    const uint16_t *v_base;
    const uint16_t *const *k_seq;
    const uint16_t *const *v_seq;
    uint64_t seq_stride;
    const uint32_t *pos0_dev;
    float *out;
    float *part_o;   /* [seq][kvh][split][col][HD] unnormalised O            */
    float2 *part_ml; /* [seq][kvh][split][col] (running max, sum) in log2 units */
    uint32_t pos0_host, n_rows, n_head_q, n_head_kv, kv_mul, ncols;
    uint32_t window, cap, n_splits, chunk, out_dims;
    /* balanced plan (k_splitkv_bal): plan.n_wg workgroups share the batch's
     * 32-key tiles evenly (splitkv_plan.h); wpg: KV heads per group */
    lfm_bal_cfg plan;
    uint32_t wpg;
    uint32_t *tile_prefix; /* [n_seq + 2] tiles before each sequence, then G (device positions) */
    int gate_is_logit;
    float qscale; /* scale * log2(e) */
    /* fused prologue (FUSE kernels): raw new-token K/V rows, norm weights,
     * RoPE tables (AttnBatch) */
    const float *k_new, *v_new, *q_norm_w, *k_norm_w, *cos_lut, *sin_lut;
    float eps;
    int prologue; /* LFM_PROLOGUE_FAST / LFM_PROLOGUE_TABLE */
};

__device__ __forceinline__ half8_t as_half8(u32x4_t v) { return __builtin_bit_cast(half8_t, v); }

/* Cache rows are read through global-address-space pointers: the
 * per-sequence pointers come from a table, so the compiler would otherwise
 * emit flat loads, which also count on lgkmcnt and make every LDS wait in the
 * loop wait for the next sub-tile's loads as well. */
typedef const __attribute__((address_space(1))) uint16_t *gu16_ptr;
typedef const __attribute__((address_space(1))) u32x4_t *gu32x4_ptr;
typedef const __attribute__((address_space(1))) uint8_t *gu8_ptr;

/* A pointer every lane holds the same value of, moved to scalar registers so
 * that loads from it plus a per-lane 32-bit offset use the SGPR-base
 * addressing form (no 64-bit address arithmetic per load). */
__device__ __forceinline__ gu8_ptr uniform_ptr(gu8_ptr p) {
    const uint64_t a  = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return (gu8_ptr)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
/* STREAM: non-temporal loads (the "nt" cache policy), for cache rows read
 * once.  Measured on MI355X with rotated copies larger than the 256 MB MALL:
 * single-row decode kernels (one 16-column tile) run faster with them --
 * B64 x 8192 (32q/8kv d64) 186.9 -> 170 us, ragged B64 100.2 -> 92.3 us,
 * LFM3 full B32 x 32768 374.8 -> 346.5 us, SWA ring 11.0 -> 10.6 us -- while
 * the 8-row verify kernel (two tiles) runs slower, 37.0 -> 40.7 us at
 * B16 x 4104, so it keeps the default policy. */
template <bool STREAM>
__device__ __forceinline__ u32x4_t load16(gu16_ptr p) {
    if constexpr (STREAM) return __builtin_nontemporal_load(reinterpret_cast<gu32x4_ptr>(p));
    else return *reinterpret_cast<gu32x4_ptr>(p);
}

__device__ __forceinline__ float4_t mfma(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

/* LDS ordering between the lanes of one wave: each wave owns its V tile,
 * so no workgroup barrier is needed; wait for this wave's LDS traffic and
 * keep the compiler from moving LDS accesses across this point. */
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f); /* lgkmcnt(0) */
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float gate_value(const float *gate, size_t idx, int is_logit) {
    if (!gate) return 1.0f;
    const float g = gate[idx];
    return is_logit ? 1.0f / (1.0f + expf(-g)) : g;
}
/* The same in two halves: the load, issued where a kernel starts so that its
 * memory round trip overlaps the kernel's work instead of delaying the
 * output, and the sigmoid where the value is used. */
__device__ __forceinline__ float gate_raw(const float *gate, size_t idx) { return gate ? gate[idx] : 1.0f; }
__device__ __forceinline__ float gate_apply(float raw, const float *gate, int is_logit) {
    return (gate && is_logit) ? 1.0f / (1.0f + expf(-raw)) : raw;
}

/* Sum of squares of one head held in MFMA fragment order (lane (l16, g)
 * holds dims 32*st + 8*g + j), added in the order of the reference's AVX2
 * kernels so the normalised rows are bit-identical to theirs; the result is
 * returned on every lane of the l16 group.
 *   HD 64 (lfm2_qk_norm_rope_avx2, tools/lfm2_kernels_fast.c:443-449): per
 *   8-lane column j, ss0 = x[j]^2 + x[32+j]^2, ss1 = x[8+j]^2 + x[40+j]^2,
 *   ss0 = fma(x[16+j], ., fma(x[48+j], ., ss0)), ss1 likewise with 24/56,
 *   t[j] = ss0 + ss1, then ((t0+t4) + (t2+t6)) + ((t1+t5) + (t3+t7)).
 *   HD 128 (lfm3_qk_norm_rope_128_avx2, tools/lfm3_engine.c:480-494): per
 *   column j, fma chains ss0 over dims 16k + j and ss1 over 16k + 8 + j,
 *   k = 0..7, s[j] = ss0 + ss1, then ((s0+s4) + (s1+s5)) + ((s2+s6) + (s3+s7)).
 * Dims 16k + j alternate between lanes g and g + 2, so the chains hop
 * between the two halves of the wave. */
template <int HD>
__device__ __forceinline__ float sumsq_ref_order(const float (&x)[HD / 32][8], int g) {
#pragma clang fp contract(off)
    float t[8];
    if constexpr (HD == 64) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float a = x[0][j], b = x[1][j];
            const float v = a * a + b * b;                    /* g 0: ss0, g 1: ss1 (first terms) */
            const float w = __shfl_xor(v, 32);                /* to g 2 / g 3                     */
            const float u = __builtin_fmaf(a, a, __builtin_fmaf(b, b, w)); /* g 2: ss0, g 3: ss1 */
            t[j]          = u + __shfl_xor(u, 16);            /* g 2, 3: ss0 + ss1                */
        }
        const float T = ((t[0] + t[4]) + (t[2] + t[6])) + ((t[1] + t[5]) + (t[3] + t[7]));
        const float o = __shfl_xor(T, 32);
        return g >= 2 ? T : o;
    } else {
        static_assert(HD == 128, "reference summation order is defined for head_dim 64 and 128");
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float acc = 0.0f;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const float xx = x[st][j];
                if (g < 2) acc = __builtin_fmaf(xx, xx, acc); /* dims 32 st + j (+8)        */
                acc = __shfl_xor(acc, 32);
                if (g >= 2) acc = __builtin_fmaf(xx, xx, acc); /* dims 32 st + 16 + j (+8)  */
                acc = __shfl_xor(acc, 32);
            }
            t[j] = acc + __shfl_xor(acc, 16); /* g 0, 1: ss0 + ss1 */
        }
        const float T = ((t[0] + t[4]) + (t[1] + t[5])) + ((t[2] + t[6]) + (t[3] + t[7]));
        const float o = __shfl_xor(T, 32);
        return g < 2 ? T : o;
    }
}

/* Mean of squares of one head in the order of lfm2_rmsnorm
 * (tools/lfm2_forward.c:669-684), the norm of the production LFM2 prologue
 * (LFM_PROLOGUE_TABLE): column j is a fused multiply-add chain over dims
 * 8k + j, k = 0 .. HD/8 - 1 in order, and the eight columns are then added
 * in order in double; the result is (float)(sum / HD).  Dim 8k + j sits in
 * fragment k / 4 of lane group g = k % 4, so the chain passes from group to
 * group: at each step every lane forms fma(x, x, acc) with its own x and the
 * value of group k % 4 is broadcast to the four lanes of the column.
 * Returned on every lane. */
template <int HD>
__device__ __forceinline__ float meansq_table_order(const float (&x)[HD / 32][8], int l16) {
#pragma clang fp contract(off)
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < HD / 32; ++st)
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[j] = __shfl(__builtin_fmaf(x[st][j], x[st][j], acc[j]), l16 + 16 * gg);
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += (double)acc[j];
    return (float)(ss / (double)HD);
}

/* QK-RMSNorm + NeoX RoPE of one head held in MFMA fragment order: lane
 * (l16, g) holds dims 32*st + 8*g + j (st < HD/32, j < 8) of the head of
 * its column, and the four lanes g = 0..3 of an l16 hold the whole head.
 * x <- (x * irms) * w with irms = 1/sqrtf(sum(x^2)/HD + eps) (skipped when
 * norm_w is null), then pairs (d, d + HD/2) -- which sit in fragments st and
 * st + HD/64 of the same lane -- rotate by the table row of position `pos`:
 * lo' = fma(lo, c, -(hi*s)), hi' = fma(hi, c, lo*s).  The arithmetic of the
 * prologue kernel and of the reference's AVX2 kernels
 * (tools/lfm2_kernels_fast.c:403-497, tools/lfm3_engine.c:463-525), sum of
 * squares included.  Every lane of the wave must call it (cross-lane sums). */
__device__ __forceinline__ void load8(const float *p, float (&x)[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

template <int HD>
__device__ __forceinline__ void norm_rope_frag(float (&x)[HD / 32][8], uint32_t pos, const float *norm_w, float eps,
                                               const float *cos_lut, const float *sin_lut, int g, int prologue) {
    constexpr int NS = HD / 32, HALF = HD / 2;
    if (norm_w) {
        const float mean = prologue == LFM_PROLOGUE_TABLE ? meansq_table_order<HD>(x, (int)(threadIdx.x & 15u))
                                                          : sumsq_ref_order<HD>(x, g) / (float)HD;
        const float irms = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            float w[8];
            load8(norm_w + 32 * st + 8 * g, w);
#pragma unroll
            for (int j = 0; j < 8; ++j) x[st][j] = (x[st][j] * irms) * w[j];
        }
    }
    const float *cr = cos_lut + (size_t)pos * HALF;
    const float *sr = sin_lut + (size_t)pos * HALF;
#pragma unroll
    for (int st = 0; st < NS / 2; ++st) {
        float c[8], sn[8];
        load8(cr + 32 * st + 8 * g, c);
        load8(sr + 32 * st + 8 * g, sn);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float lo = x[st][j], hi = x[st + NS / 2][j];
            x[st][j]          = __builtin_fmaf(lo, c[j], -(hi * sn[j]));
            x[st + NS / 2][j] = __builtin_fmaf(hi, c[j], lo * sn[j]);
        }
    }
}

/* Two fp32 values stored as RNE fp16 (packed).  Each value is first
 * materialised in fp32 (the reference stores fp32 results with
 * _mm256_cvtps_ph): the barrier keeps the compiler from fusing a producing
 * fma with the conversion into v_fma_mixlo_f16, whose single rounding
 * differs on ties. */
__device__ __forceinline__ uint32_t pack_rne(float a, float b) {
    asm volatile("" : "+v"(a));
    asm volatile("" : "+v"(b));
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

__device__ __forceinline__ u32x4_t pack8_rne(const float (&x)[8]) {
    u32x4_t w;
    w[0] = pack_rne(x[0], x[1]);
    w[1] = pack_rne(x[2], x[3]);
    w[2] = pack_rne(x[4], x[5]);
    w[3] = pack_rne(x[6], x[7]);
    return w;
}

/* Keys [lo, last] that the rows of sequence s attend (their union). */
struct SeqKeys {
    uint32_t pos0, lo, last;
};
__device__ __forceinline__ SeqKeys seq_keys(const SplitParams &P, uint32_t s) {
    SeqKeys k;
    k.pos0 = P.pos0_dev ? P.pos0_dev[s] : P.pos0_host;
    k.last = k.pos0 + P.n_rows - 1u;
    k.lo   = lfm_plan_row(k.pos0, P.window, P.cap).t_start;
    return k;
}

/* One wave: the attention of KV head kvh of sequence s over keys [kb, ke).
 * direct: the range is the sequence's whole key set, so the normalised,
 * gated output is written; otherwise the unnormalised O^T and (max, sum)
 * go to the partial slots part + column. */
template <int HD, int NT, bool FUSE>
__device__ __forceinline__ void run_segment(const SplitParams &P, uint16_t *vt, uint16_t *fresh, uint32_t s,
                                            uint32_t pos0, uint32_t kvh, uint32_t kb, uint32_t ke, bool direct,
                                            size_t part) {
    constexpr int NS  = HD / 32; /* MFMA k-steps of Q.K^T (32 dims each)          */
    constexpr int NM  = HD / 16; /* 16-dim tiles of O^T                            */
    constexpr int NVL = HD / 16; /* 16-byte V pieces per lane per 32-key sub-tile  */
    constexpr int CH  = HD / 8;  /* 16-byte chunks per V row                       */
    constexpr int QPP = 64 / CH; /* 4-key quads covered by one pass of 64 lanes    */
    constexpr bool PSPLIT = NT == 1; /* P split hi + lo (one 16-column tile)       */
    const int lane = threadIdx.x & 63;
    const int l16  = lane & 15;
    const int g    = lane >> 4;
    /* The segment is the same for every lane, but in k_splitkv_wg and
     * k_splitkv_bal it derives from threadIdx and lane shuffles, so the
     * compiler held it in VGPRs and lowered the key loop and the fused
     * prologue's branches as divergent (EXEC-masked) code.  The head_dim-128,
     * 32-column fused instantiations of those two kernels then returned wrong
     * outputs on MI355X (up to 1.5 absolute, every plan but the grid, whose
     * segment comes from blockIdx); with the values made explicitly uniform
     * the control flow is scalar and every plan matches the oracle. */
    kb   = __builtin_amdgcn_readfirstlane(kb);
    ke   = __builtin_amdgcn_readfirstlane(ke);
    pos0 = __builtin_amdgcn_readfirstlane(pos0);
    kvh  = __builtin_amdgcn_readfirstlane(kvh);
    s    = __builtin_amdgcn_readfirstlane(s);
    const uint32_t last = pos0 + P.n_rows - 1u;

    gu16_ptr kc = (gu16_ptr)(P.k_seq ? P.k_seq[s] : P.k_base + (size_t)s * P.seq_stride);
    gu16_ptr vc = (gu16_ptr)(P.v_seq ? P.v_seq[s] : P.v_base + (size_t)s * P.seq_stride);
    const size_t row   = (size_t)P.n_head_kv * HD; /* elements per cache slot */
    kc += (size_t)kvh * HD;
    vc += (size_t)kvh * HD;

    /* ---- sub-tile loader ------------------------------------------------------
     * A sub-tile whose 32 slots are contiguous and inside [kb, ke) (every one
     * but a segment's last, or one that wraps the ring) loads from a
     * wave-uniform base pointer plus per-lane 32-bit byte offsets fixed for
     * the segment, so no per-load address arithmetic runs on the VALU; the
     * others clamp and wrap per lane. */
    uint32_t koffb[2], voffb[NVL]; /* set after the first sub-tile's loads are issued */
    auto load_tile = [&](uint32_t p0, u32x4_t (&kd)[2][NS], u32x4_t (&vd)[NVL], bool may_fast) {
        const uint32_t base = P.window ? (p0 % P.cap) : p0;
        if (may_fast && p0 + 32u <= ke && (!P.window || base + 32u <= P.cap)) {
            gu8_ptr k0 = uniform_ptr((gu8_ptr)(kc + (size_t)base * row));
            gu8_ptr v0 = uniform_ptr((gu8_ptr)(vc + (size_t)base * row));
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int st = 0; st < NS; ++st)
                    kd[kt][st] = load16<NT == 1>((gu16_ptr)(k0 + koffb[kt] + 64u * st));
#pragma unroll
            for (int j = 0; j < NVL; ++j) vd[j] = load16<NT == 1>((gu16_ptr)(v0 + voffb[j]));
            return;
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            uint32_t off = (uint32_t)(16 * kt + l16);
            if (p0 + off >= ke) off = ke - 1u - p0; /* clamp: masked later */
            uint32_t slot = base + off;
            if (P.window) { while (slot >= P.cap) slot -= P.cap; }
            gu16_ptr kp = kc + (size_t)slot * row + 8 * g;
#pragma unroll
            for (int st = 0; st < NS; ++st)
                kd[kt][st] = load16<NT == 1>(kp + 32 * st);
        }
#pragma unroll
        for (int ps = 0; ps < HD / 64; ++ps) {
            const int quad = ps * QPP + lane / CH;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t off = (uint32_t)(4 * quad + i);
                if (p0 + off >= ke) off = ke - 1u - p0;
                uint32_t slot = base + off;
                if (P.window) { while (slot >= P.cap) slot -= P.cap; }
                vd[ps * 4 + i] = load16<NT == 1>(vc + (size_t)slot * row + 8 * (lane % CH));
            }
        }
    };

    /* the first sub-tile is in flight while the query fragments are built */
    const uint32_t nsub = (ke - kb + 31u) / 32u;
    u32x4_t kA[2][NS], vA[NVL], kB[2][NS], vB[NVL];
    load_tile(kb, kA, vA, false);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) koffb[kt] = (uint32_t)(((16 * kt + l16) * row + 8 * g) * sizeof(uint16_t));
#pragma unroll
    for (int ps = 0; ps < HD / 64; ++ps)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            voffb[ps * 4 + i] =
                (uint32_t)(((4 * (ps * QPP + lane / CH) + i) * row + 8 * (lane % CH)) * sizeof(uint16_t));

    /* ---- per-column row bounds and Q fragments ------------------------------ */
    uint32_t col_lo[NT], col_hi[NT];
    half8_t qh[NT][NS], ql[NT][NS];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t n = (uint32_t)(l16 + 16 * nt);
        col_lo[nt] = 0xFFFFFFFFu; /* padding column: every key masked */
        col_hi[nt] = 0u;
        float x[NS][8];
        const bool live = n < P.ncols;
        uint32_t abs    = pos0;
        if (live) {
            const uint32_t r = n / P.kv_mul;
            const uint32_t h = kvh * P.kv_mul + (n - r * P.kv_mul);
            abs              = pos0 + r;
            col_lo[nt]       = lfm_plan_row(abs, P.window, P.cap).t_start;
            col_hi[nt]       = abs;
            const float *qp  = P.q + (((size_t)s * P.n_rows + r) * P.n_head_q + h) * HD + 8 * g;
#pragma unroll
            for (int st = 0; st < NS; ++st) load8(qp + 32 * st, x[st]);
        } else {
#pragma unroll
            for (int st = 0; st < NS; ++st)
#pragma unroll
                for (int j = 0; j < 8; ++j) x[st][j] = 0.0f;
        }
        /* fused prologue: the raw query is normalised and rotated here, by
         * every wave that reads it (all lanes take part in the sums) */
        if constexpr (FUSE) norm_rope_frag<HD>(x, abs, P.q_norm_w, P.eps, P.cos_lut, P.sin_lut, g, P.prologue);
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                /* xs is rounded to fp32 before the split: otherwise the
                 * compiler may fuse the product into a mixed-precision fma
                 * that rounds x*qscale - hi straight to fp16 in some
                 * instantiations and not others, and the lo parts of the
                 * fused and plain kernels then differ on double-rounding
                 * ties (about one element in 8000).  With xs rounded, xs - hi
                 * is exact and lo is its only rounding. */
                float xs = x[st][j] * P.qscale;
                asm volatile("" : "+v"(xs));
                const _Float16 hi = (_Float16)xs;
                qh[nt][st][j]     = hi;
                ql[nt][st][j]     = (_Float16)(xs - (float)hi);
            }
    }
    /* keys every real column may see without a per-key test */
    const uint32_t free_lo = lfm_plan_row(last, P.window, P.cap).t_start;
    const uint32_t free_hi = min(pos0, ke - 1u);


    /* ---- fused prologue: the rows of this call's positions -------------------
     * Keys >= pos0 are the new tokens.  Before the key loop, the wave whose
     * range [kb, ke) holds new keys builds those rows from the raw k/v
     * (normalised, rotated, RNE fp16), stores them at their cache slots and
     * stages them in its LDS area `fresh` ([n_rows][HD] K, then V).  Each new
     * key lies in exactly one segment of the plan, so each row is stored once,
     * and no other wave reads those bytes in this launch.  In the loop, the
     * sub-tiles that reach pos0 take those rows from LDS in place of what was
     * loaded from the slots (lanes clamped past ke take the last key's row
     * too, so no stale slot content enters the product); the loop itself
     * issues no extra global memory operations. */
    const bool has_fresh = FUSE && ke > pos0;
    if constexpr (FUSE) {
        if (has_fresh) {
            uint16_t *kw = const_cast<uint16_t *>(P.k_seq ? P.k_seq[s] : P.k_base + (size_t)s * P.seq_stride) +
                           (size_t)kvh * HD;
            uint16_t *vw = const_cast<uint16_t *>(P.v_seq ? P.v_seq[s] : P.v_base + (size_t)s * P.seq_stride) +
                           (size_t)kvh * HD;
            const uint32_t r0 = max(kb, pos0) - pos0, r1 = ke - pos0; /* rows of this segment */
            for (uint32_t rb = r0; rb < r1; rb += 16u) {
                const uint32_t r  = rb + (uint32_t)l16;
                const bool real   = r < r1;
                float x[NS][8];
                if (real) {
                    const float *kp = P.k_new + (((size_t)s * P.n_rows + r) * P.n_head_kv + kvh) * HD + 8 * g;
#pragma unroll
                    for (int st = 0; st < NS; ++st) load8(kp + 32 * st, x[st]);
                } else {
#pragma unroll
                    for (int st = 0; st < NS; ++st)
#pragma unroll
                        for (int j = 0; j < 8; ++j) x[st][j] = 0.0f;
                }
                norm_rope_frag<HD>(x, real ? pos0 + r : pos0, P.k_norm_w, P.eps, P.cos_lut, P.sin_lut, g,
                                   P.prologue);
                if (real) {
                    const size_t off = (size_t)lfm_slot_of(pos0 + r, P.window, P.cap) * row + 8 * g;
#pragma unroll
                    for (int st = 0; st < NS; ++st) {
                        const u32x4_t w = pack8_rne(x[st]);
                        *reinterpret_cast<u32x4_t *>(kw + off + 32 * st)                        = w;
                        *reinterpret_cast<u32x4_t *>(fresh + (size_t)r * HD + 8 * g + 32 * st) = w;
                    }
                }
            }
            for (uint32_t e = r0 * CH + (uint32_t)lane; e < r1 * CH; e += 64u) {
                const uint32_t r = e / CH, c = e % CH;
                float x[8];
                load8(P.v_new + (((size_t)s * P.n_rows + r) * P.n_head_kv + kvh) * HD + 8 * c, x);
                const u32x4_t w = pack8_rne(x);
                *reinterpret_cast<u32x4_t *>(vw + (size_t)lfm_slot_of(pos0 + r, P.window, P.cap) * row + 8 * c) = w;
                *reinterpret_cast<u32x4_t *>(fresh + (size_t)(P.n_rows + r) * HD + 8 * c)                     = w;
            }
            wave_lds_sync();
        }
    }
    /* the staged rows in place of the slots' contents, for the lanes whose
     * (clamped) key is >= pos0 */
    auto patch_new_rows = [&](uint32_t p0, u32x4_t (&kd)[2][NS], u32x4_t (&vd)[NVL]) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            uint32_t key = p0 + (uint32_t)(16 * kt + l16);
            if (key >= ke) key = ke - 1u;
            if (key >= pos0) {
#pragma unroll
                for (int st = 0; st < NS; ++st)
                    kd[kt][st] = *reinterpret_cast<const u32x4_t *>(fresh + (size_t)(key - pos0) * HD + 8 * g + 32 * st);
            }
        }
#pragma unroll
        for (int ps = 0; ps < HD / 64; ++ps) {
            const int quad = ps * QPP + lane / CH;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t key = p0 + (uint32_t)(4 * quad + i);
                if (key >= ke) key = ke - 1u;
                if (key >= pos0)
                    vd[ps * 4 + i] = *reinterpret_cast<const u32x4_t *>(
                        fresh + (size_t)(P.n_rows + key - pos0) * HD + 8 * (lane % CH));
            }
        }
    };

    float4_t oacc[NM][NT];
    float mrun[NT], lrun[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        mrun[nt] = kNegBig;
        lrun[nt] = 0.0f;
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] = (float4_t)0.0f;
    }

    /* One 32-key sub-tile: V to LDS, S^T, online softmax, O^T update.
     * V of a sub-tile goes to the wave's LDS area row-major, each 64-dim half
     * of a row as 128 B with its 16-B chunks XOR-swizzled by row & 7; the
     * P.V operand V^T then comes from transposing reads (ds_read_b64_tr_b16),
     * bank-conflict free, with no VALU transpose.
     * Lane (l16, g) reads row 4g + l16/4 of a 16-key half at dims
     * 16 mt + 4 (l16 % 4), in the key order of P's accumulator layout. */
    uint8_t *vrow = reinterpret_cast<uint8_t *>(vt);
    /* this lane stores rows 4q + i, i < 4 (q = lane / CH, plus QPP per pass)
     * of 16-byte chunk c: row 4q + i holds it at slot c ^ ((4q + i) & 7) =
     * (c ^ 4 (q & 1)) ^ i, 128 B apart */
    const uint32_t vsq = (uint32_t)(lane / CH), vsc = (uint32_t)(lane % CH);
    const uint32_t vst = (vsc >> 3) * 4096u + vsq * 512u;
    const uint32_t vsw = (vsc & 7u) ^ (4u * (vsq & 1u));
    auto vst_off = [&](int j) {
        const uint32_t i = (uint32_t)(j & 3);
        return vst + (uint32_t)(j >> 2) * (uint32_t)QPP * 512u + i * 128u + 16u * (vsw ^ i);
    };
    /* QPP is a multiple of 4 (rows 16 or 32 apart), so later passes keep the swizzle */
    static_assert(QPP % 4 == 0, "V store swizzle assumes whole 4-quad groups per pass");
    /* the transposing read of dims 16 mt'..16 mt' + 15 (mt' = mt % 4) of row
     * vr: chunk 2 mt' + ((l16 >> 1) & 1) at slot (2 mt' + b) ^ (vr & 7) = 2 mt'
     * ^ (b ^ (vr & 7)), so the read address is vtr ^ (32 mt') */
    const uint32_t vr  = (uint32_t)(4 * g + (l16 >> 2));
    const uint32_t vtr = vr * 128u + 16u * ((uint32_t)((l16 >> 1) & 1) ^ (vr & 7u)) + 8u * (uint32_t)(l16 & 1);
    auto process = [&](uint32_t p0, const u32x4_t (&kcur)[2][NS], const u32x4_t (&vcur)[NVL]) {
        wave_lds_sync(); /* previous sub-tile's transposing V reads are done */
#pragma unroll
        for (int j = 0; j < NVL; ++j)
            *reinterpret_cast<u32x4_t *>(vrow + vst_off(j)) =
                vcur[j];

        /* S^T = K . Q^T (log2 units) */
        float4_t sacc[2][NT];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                float4_t acc = (float4_t)0.0f;
#pragma unroll
                for (int st = 0; st < NS; ++st) {
                    acc = mfma(as_half8(kcur[kt][st]), qh[nt][st], acc);
                    acc = mfma(as_half8(kcur[kt][st]), ql[nt][st], acc);
                }
                sacc[kt][nt] = acc;
            }

        /* masks: only sub-tiles touching a row bound or the split end */
        const bool need_mask = (p0 < free_lo) || (p0 + 31u > free_hi);
        if (need_mask) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t key = p0 + (uint32_t)(16 * kt + 4 * g + i);
                        const bool ok = key < ke && key >= col_lo[nt] && key <= col_hi[nt];
                        if (!ok) sacc[kt][nt][i] = -INFINITY;
                    }
        }

        /* online softmax; P^T fragments.  Lazy running max: m is raised only
         * when a sub-tile's column max exceeds it by more than kLazyMax (so
         * p <= 2^kLazyMax), and O is rescaled only then; the first sub-tile
         * with an unmasked key sets m (from the kNegBig sentinel).  With one
         * 16-column tile P is split hi + lo like Q (the MFMAs are free in
         * this HBM-bound kernel); with more, P enters as one fp16 value
         * (relative rounding 2^-11 per weight). */
        half8_t ph[NT], pl[NT];
        float alpha_nt[NT];
        bool rose = false;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float mx = fmaxf(fmaxf(fmaxf(sacc[0][nt][0], sacc[0][nt][1]), fmaxf(sacc[0][nt][2], sacc[0][nt][3])),
                             fmaxf(fmaxf(sacc[1][nt][0], sacc[1][nt][1]), fmaxf(sacc[1][nt][2], sacc[1][nt][3])));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool raise  = mx > mrun[nt] + kLazyMax;
            const float mnew  = raise ? mx : mrun[nt];
            const float alpha = raise ? __builtin_amdgcn_exp2f(mrun[nt] - mnew) : 1.0f;
            rose             |= raise;
            alpha_nt[nt]      = alpha;
            mrun[nt]          = mnew;
            float psum        = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p      = __builtin_amdgcn_exp2f(sacc[kt][nt][i] - mnew);
                    psum              += p;
                    const _Float16 hi  = (_Float16)p;
                    ph[nt][4 * kt + i] = hi;
                    if constexpr (PSPLIT) pl[nt][4 * kt + i] = (_Float16)(p - (float)hi);
                }
            lrun[nt] = lrun[nt] * alpha + psum;
        }
        if (__builtin_amdgcn_ballot_w64(rose) != 0ull) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] *= alpha_nt[nt];
        }

        wave_lds_sync(); /* V of this sub-tile is in LDS */
        /* O^T += V^T . P^T */
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) {
            const uint8_t *vh   = vrow + (mt >> 2) * 4096u;
            const uint32_t o    = vtr ^ (32u * (uint32_t)(mt & 3));
            const half4v_t lo   = lds_read_tr(vh + o);
            const half4v_t hi   = lds_read_tr(vh + 16u * 128u + o);
            const half8_t av    = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                oacc[mt][nt] = mfma(av, ph[nt], oacc[mt][nt]);
                if constexpr (PSPLIT) oacc[mt][nt] = mfma(av, pl[nt], oacc[mt][nt]);
            }
        }
    };

    /* The last two sub-tiles of a segment in one step (one-tile kernels):
     * both score sets first, one column max and one lazy-max decision for
     * the 64 keys, then P.V of each sub-tile through the wave's V tile in
     * turn.  Segments of two sub-tiles (config 1, the LFM3 window ring) are
     * mostly this dependent chain, which runs once instead of twice. */
    auto process2 = [&](uint32_t p0, const u32x4_t (&ka)[2][NS], const u32x4_t (&va)[NVL],
                        const u32x4_t (&kb)[2][NS], const u32x4_t (&vb)[NVL]) {
        wave_lds_sync(); /* previous sub-tile's transposing V reads are done */
#pragma unroll
        for (int j = 0; j < NVL; ++j)
            *reinterpret_cast<u32x4_t *>(vrow + vst_off(j)) =
                va[j];
        float4_t sacc[2][2]; /* [sub-tile][16-key half] */
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                float4_t acc = (float4_t)0.0f;
#pragma unroll
                for (int st = 0; st < NS; ++st) {
                    const half8_t kf = as_half8(u ? kb[kt][st] : ka[kt][st]);
                    acc = mfma(kf, qh[0][st], acc);
                    acc = mfma(kf, ql[0][st], acc);
                }
                sacc[u][kt] = acc;
            }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t pu = p0 + 32u * (uint32_t)u;
            if ((pu < free_lo) || (pu + 31u > free_hi)) {
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t key = pu + (uint32_t)(16 * kt + 4 * g + i);
                        const bool ok      = key < ke && key >= col_lo[0] && key <= col_hi[0];
                        if (!ok) sacc[u][kt][i] = -INFINITY;
                    }
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                mx = fmaxf(mx, fmaxf(fmaxf(sacc[u][kt][0], sacc[u][kt][1]), fmaxf(sacc[u][kt][2], sacc[u][kt][3])));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const bool raise  = mx > mrun[0] + kLazyMax;
        const float mnew  = raise ? mx : mrun[0];
        const float alpha = raise ? __builtin_amdgcn_exp2f(mrun[0] - mnew) : 1.0f;
        mrun[0]           = mnew;
        half8_t ph[2], pl[2];
        float psum = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pv    = __builtin_amdgcn_exp2f(sacc[u][kt][i] - mnew);
                    psum             += pv;
                    const _Float16 hi = (_Float16)pv;
                    ph[u][4 * kt + i] = hi;
                    pl[u][4 * kt + i] = (_Float16)(pv - (float)hi);
                }
        lrun[0] = lrun[0] * alpha + psum;
        if (__builtin_amdgcn_ballot_w64(raise) != 0ull) {
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) oacc[mt][0] *= alpha;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1) {
                wave_lds_sync(); /* the first sub-tile's transposing reads are done */
#pragma unroll
                for (int j = 0; j < NVL; ++j)
                    *reinterpret_cast<u32x4_t *>(vrow + vst_off(j)) = vb[j];
            }
            wave_lds_sync(); /* V of this sub-tile is in LDS */
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const uint8_t *vh = vrow + (mt >> 2) * 4096u;
                const uint32_t o  = vtr ^ (32u * (uint32_t)(mt & 3));
                const half4v_t lo = lds_read_tr(vh + o);
                const half4v_t hi = lds_read_tr(vh + 16u * 128u + o);
                const half8_t av  = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                oacc[mt][0]       = mfma(av, ph[u], oacc[mt][0]);
                oacc[mt][0]       = mfma(av, pl[u], oacc[mt][0]);
            }
        }
    };

    /* two register buffers; the loads of sub-tile i+1 are in flight while
     * sub-tile i is consumed.  The loop body issues its loads unconditionally
     * and the last one or two sub-tiles are peeled: with a conditional load
     * inside the loop the compiler's wait counts had to cover the path that
     * skipped it, so each sub-tile waited for the next one's loads as well
     * (vmcnt(0)).  Measured on MI355X: headline 192.4 -> 190.0 us, verify
     * 41.7 -> 39.7 us, LFM3 SWA 10.6 -> 10.3 us, outputs bit-identical. */
    /* sub-tile at p0 with its new rows substituted (FUSE), then consumed */
    auto consume = [&](uint32_t p0, u32x4_t (&kd)[2][NS], u32x4_t (&vd)[NVL]) {
        if constexpr (FUSE) {
            if (has_fresh && p0 + 31u >= pos0) patch_new_rows(p0, kd, vd);
        }
        process(p0, kd, vd);
    };
    auto consume2 = [&](uint32_t p0, u32x4_t (&ka)[2][NS], u32x4_t (&va)[NVL], u32x4_t (&kb)[2][NS],
                        u32x4_t (&vb)[NVL]) {
        if constexpr (FUSE) {
            if (has_fresh && p0 + 31u >= pos0) patch_new_rows(p0, ka, va);
            if (has_fresh && p0 + 63u >= pos0) patch_new_rows(p0 + 32u, kb, vb);
        }
        process2(p0, ka, va, kb, vb);
    };
    uint32_t it = 0;
    for (; it + 2u < nsub; it += 2u) {
        const uint32_t p0 = kb + 32u * it;
        load_tile(p0 + 32u, kB, vB, true);
        consume(p0, kA, vA);
        load_tile(p0 + 64u, kA, vA, true);
        consume(p0 + 32u, kB, vB);
    }
    {
        const uint32_t p0 = kb + 32u * it;
        if (it + 1u < nsub) {
            load_tile(p0 + 32u, kB, vB, true);
            if constexpr (NT == 1) {
                consume2(p0, kA, vA, kB, vB);
            } else {
                consume(p0, kA, vA);
                consume(p0 + 32u, kB, vB);
            }
        } else {
            consume(p0, kA, vA);
        }
    }

    /* ---- epilogue ---------------------------------------------------------- */
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        float lt = lrun[nt] + __shfl_xor(lrun[nt], 16);
        lt += __shfl_xor(lt, 32);
        const uint32_t n = (uint32_t)(l16 + 16 * nt);
        if (n >= P.ncols) continue;
        const uint32_t r = n / P.kv_mul;
        const uint32_t h = kvh * P.kv_mul + (n - r * P.kv_mul);
        if (direct) {
            const size_t orow = ((size_t)s * P.n_rows + r) * P.n_head_q + h;
            const float gv    = gate_value(P.gate, orow, P.gate_is_logit);
            const float inv   = (lt > 0.0f) ? gv / lt : 0.0f;
            float *op         = P.out + orow * HD;
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const uint32_t d = (uint32_t)(16 * mt + 4 * g);
                if (d < P.out_dims) {
                    float4 v = make_float4(oacc[mt][nt][0] * inv, oacc[mt][nt][1] * inv,
                                           oacc[mt][nt][2] * inv, oacc[mt][nt][3] * inv);
                    *reinterpret_cast<float4 *>(op + d) = v;
                }
            }
        } else {
            float *po = P.part_o + (part + n) * HD;
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const uint32_t d = (uint32_t)(16 * mt + 4 * g);
                *reinterpret_cast<float4 *>(po + d) =
                    make_float4(oacc[mt][nt][0], oacc[mt][nt][1], oacc[mt][nt][2], oacc[mt][nt][3]);
            }
            if (g == 0) P.part_ml[part + n] = make_float2(mrun[nt], lt);
        }
    }
}

/* ---- LDS-streamed segments (no fused prologue) ------------------------------
 * run_segment keeps one 32-key sub-tile in flight per wave, in registers, so
 * a wave's throughput is one sub-tile per memory round trip; with two 16-
 * column tiles (speculative verify) its registers leave no room for a
 * second.  Here both K and V of each sub-tile move from global memory
 * straight into a ring of DMA_NBUF sub-tiles in the wave's own LDS area
 * (global_load_lds_dwordx4: no registers held while a load is in flight),
 * three sub-tiles ahead of the one being consumed, and the wave reads K
 * fragments (ds_read_b128) and the transposed V operand (ds_read_b64_tr_b16)
 * from there.  Each sub-tile is K then V, each HD / 64 halves of [32
 * keys][128 B], the 16-B chunks of row r XOR-swizzled by r & 7 (the layout
 * run_segment stores V in).  The loads are inline assembly, invisible to the
 * compiler's wait counting, so the waits are explicit: every vector memory
 * operation in the key loop is one of these (dma_per_sub per sub-tile), and
 * before sub-tile t is read the wave waits until only the sub-tiles issued
 * after it (at most 3) remain outstanding.  Waves never read each other's
 * areas, so no workgroup barrier runs.  The default for two 16-column tiles
 * at head_dim 64 (verify rows); the one-tile forms measured slower than
 * run_segment (head_dim 64 B64 x 8192: 162.4-163.6 vs 158.4-159.7 us per
 * step; head_dim 128 B32 x 32768: 336.3-339.2 vs 333.0-333.2 us). */
constexpr int DMA_NBUF  = 4; /* ring slots per wave      */
constexpr int DMA_AHEAD = 3; /* sub-tiles in flight ahead */
static_assert(DMA_AHEAD < DMA_NBUF, "the slot being fetched must not be the one being read");
/* bytes per slot (K, then V: 32 keys x HD halfs each) and 1-KB loads per sub-tile */
template <int HD> constexpr int dma_tile() { return 2 * 32 * HD * 2; }
template <int HD> constexpr int dma_per_sub() { return 8 * (HD / 64); }

/* 16 B per lane into LDS: lane l writes [lds + 16 l, lds + 16 l + 16) (lds in
 * M0), from a wave-uniform base plus a 32-bit per-lane byte offset, or from
 * a per-lane address; STREAM: the non-temporal cache policy. */
template <bool STREAM>
__device__ __forceinline__ void dma16(uint32_t voff, gu8_ptr sbase, uint32_t lds) {
    if constexpr (STREAM)
        asm volatile("global_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
    else
        asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}
template <bool STREAM>
__device__ __forceinline__ void dma16(gu8_ptr addr, uint32_t lds) {
    if constexpr (STREAM) asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(addr), "{m0}"(lds) : "memory");
    else asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(addr), "{m0}"(lds) : "memory");
}

/* Wait until at most `younger` sub-tiles' loads (wave-uniform, <= 3) are
 * outstanding: dma_per_sub<HD>() loads each. */
template <int HD>
__device__ __forceinline__ void dma_wait(uint32_t younger) {
    static_assert(DMA_AHEAD == 3, "wait counts below");
    if constexpr (HD == 64) {
        if (younger >= 3u) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
        else if (younger == 2u) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else if (younger == 1u) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        static_assert(HD == 128, "head_dim 64 or 128");
        if (younger >= 3u) asm volatile("s_waitcnt vmcnt(48)" ::: "memory");
        else if (younger == 2u) asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
        else if (younger == 1u) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

template <int HD, int NT>
__device__ __forceinline__ void run_segment_dma(const SplitParams &P, uint8_t *ring, uint32_t s, uint32_t pos0,
                                                uint32_t kvh, uint32_t kb, uint32_t ke, bool direct, size_t part) {
    constexpr int NH          = HD / 64; /* 64-dim halves of a row: 4-KB K and V parts each */
    constexpr int NS          = HD / 32; /* MFMA k-steps of Q.K^T */
    constexpr int NM          = HD / 16; /* 16-dim tiles of O^T   */
    constexpr uint32_t TILE   = (uint32_t)dma_tile<HD>();
    constexpr bool PSPLIT     = NT == 1;
    constexpr bool STREAM     = NT == 1; /* as load16's policy in run_segment */
    const int lane = threadIdx.x & 63;
    const int l16  = lane & 15;
    const int g    = lane >> 4;
    kb   = __builtin_amdgcn_readfirstlane(kb);
    ke   = __builtin_amdgcn_readfirstlane(ke);
    pos0 = __builtin_amdgcn_readfirstlane(pos0);
    kvh  = __builtin_amdgcn_readfirstlane(kvh);
    s    = __builtin_amdgcn_readfirstlane(s);
    const uint32_t last = pos0 + P.n_rows - 1u;

    gu16_ptr kc = (gu16_ptr)(P.k_seq ? P.k_seq[s] : P.k_base + (size_t)s * P.seq_stride);
    gu16_ptr vc = (gu16_ptr)(P.v_seq ? P.v_seq[s] : P.v_base + (size_t)s * P.seq_stride);
    const size_t row = (size_t)P.n_head_kv * HD;
    kc += (size_t)kvh * HD;
    vc += (size_t)kvh * HD;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)ring;

    /* lane l's 16 B of 1-KB piece e of 64-dim half h of a K or V sub-tile:
     * row r = 8 e + l / 8, LDS chunk slot l % 8 of the half, holding the row's
     * chunk 8 h + ((l % 8) ^ swizzle(r)) */
    uint32_t drow[4], dchunk[4], doff[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        drow[e]   = 8u * (uint32_t)e + ((uint32_t)lane >> 3);
        dchunk[e] = ((uint32_t)lane & 7u) ^ (drow[e] & 7u);
        doff[e]   = (uint32_t)((drow[e] * row + 8u * dchunk[e]) * sizeof(uint16_t));
    }
    const uint32_t nsub = (ke - kb + 31u) / 32u;
    auto fetch = [&](uint32_t t) {
        const uint32_t p0   = kb + 32u * t;
        const uint32_t dst  = ring_lds + (t % (uint32_t)DMA_NBUF) * TILE;
        const uint32_t base = P.window ? (p0 % P.cap) : p0;
        if (p0 + 32u <= ke && (!P.window || base + 32u <= P.cap)) {
            gu8_ptr k0 = uniform_ptr((gu8_ptr)(kc + (size_t)base * row));
            gu8_ptr v0 = uniform_ptr((gu8_ptr)(vc + (size_t)base * row));
#pragma unroll
            for (int h = 0; h < NH; ++h)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    dma16<STREAM>(doff[e] + 128u * (uint32_t)h, k0, dst + 4096u * (uint32_t)h + 1024u * (uint32_t)e);
#pragma unroll
            for (int h = 0; h < NH; ++h)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    dma16<STREAM>(doff[e] + 128u * (uint32_t)h, v0,
                                  dst + 4096u * (uint32_t)(NH + h) + 1024u * (uint32_t)e);
            return;
        }
        /* a segment's last sub-tile, or one that wraps the ring: rows past
         * ke read the last key's row (masked), slots wrap */
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t off = drow[e];
            if (p0 + off >= ke) off = ke - 1u - p0;
            uint32_t slot = base + off;
            if (P.window) { while (slot >= P.cap) slot -= P.cap; }
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const size_t eo = (size_t)slot * row + 64u * (uint32_t)h + 8u * dchunk[e];
                dma16<STREAM>((gu8_ptr)(kc + eo), dst + 4096u * (uint32_t)h + 1024u * (uint32_t)e);
                dma16<STREAM>((gu8_ptr)(vc + eo), dst + 4096u * (uint32_t)(NH + h) + 1024u * (uint32_t)e);
            }
        }
    };
    /* the first sub-tiles are in flight while the query fragments are built
     * (a previous segment of this wave has finished reading the ring) */
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (uint32_t t = 0; t < (uint32_t)DMA_AHEAD; ++t)
        if (t < nsub) fetch(t);

    /* ---- per-column row bounds and Q fragments (as run_segment) ------------- */
    uint32_t col_lo[NT], col_hi[NT];
    half8_t qh[NT][NS], ql[NT][NS];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t n = (uint32_t)(l16 + 16 * nt);
        col_lo[nt] = 0xFFFFFFFFu;
        col_hi[nt] = 0u;
        float x[NS][8];
        if (n < P.ncols) {
            const uint32_t r = n / P.kv_mul;
            const uint32_t h = kvh * P.kv_mul + (n - r * P.kv_mul);
            col_lo[nt]       = lfm_plan_row(pos0 + r, P.window, P.cap).t_start;
            col_hi[nt]       = pos0 + r;
            const float *qp  = P.q + (((size_t)s * P.n_rows + r) * P.n_head_q + h) * HD + 8 * g;
#pragma unroll
            for (int st = 0; st < NS; ++st) load8(qp + 32 * st, x[st]);
        } else {
#pragma unroll
            for (int st = 0; st < NS; ++st)
#pragma unroll
                for (int j = 0; j < 8; ++j) x[st][j] = 0.0f;
        }
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float xs = x[st][j] * P.qscale;
                asm volatile("" : "+v"(xs)); /* rounded once, as in run_segment */
                const _Float16 hi = (_Float16)xs;
                qh[nt][st][j]     = hi;
                ql[nt][st][j]     = (_Float16)(xs - (float)hi);
            }
    }
    const uint32_t free_lo = lfm_plan_row(last, P.window, P.cap).t_start;
    const uint32_t free_hi = min(pos0, ke - 1u);

    float4_t oacc[NM][NT];
    float mrun[NT], lrun[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        mrun[nt] = kNegBig;
        lrun[nt] = 0.0f;
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] = (float4_t)0.0f;
    }
    /* K fragment of key 16 kt + l16, dims 32 st + 8 g: chunk 4 st + g */
    const uint32_t kswz  = (uint32_t)g ^ ((uint32_t)l16 & 7u);
    const uint32_t koff0 = (uint32_t)l16 * 128u + 16u * kswz;
    const uint32_t koff1 = (uint32_t)l16 * 128u + 16u * (kswz ^ 4u);
    const uint32_t vr    = (uint32_t)(4 * g + (l16 >> 2));
    const uint32_t vtr   = vr * 128u + 16u * ((uint32_t)((l16 >> 1) & 1) ^ (vr & 7u)) + 8u * (uint32_t)(l16 & 1);

    /* (Software pipelining this loop -- the score MFMAs of sub-tile t + 1
     * issued before the softmax and P.V of t -- measured no faster on
     * MI355X for the 8-row verify, 37.8-38.3 vs 37.6-37.9 us per step.) */
    for (uint32_t t = 0; t < nsub; ++t) {
        if (t + (uint32_t)DMA_AHEAD < nsub) {
            /* the slot being refilled held sub-tile t - 1, whose LDS reads
             * this wave has finished */
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            fetch(t + (uint32_t)DMA_AHEAD);
        }
        dma_wait<HD>(min(nsub - 1u - t, (uint32_t)DMA_AHEAD));
        const uint32_t p0  = kb + 32u * t;
        const uint8_t *kt0 = ring + (t % (uint32_t)DMA_NBUF) * TILE;
        const uint8_t *vt0 = kt0 + NH * 4096;

        /* S^T = K . Q^T (log2 units); k-step st reads 64-dim half st / 2 */
        float4_t sacc[2][NT];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            half8_t kf[NS];
#pragma unroll
            for (int st = 0; st < NS; ++st)
                kf[st] = as_half8(*reinterpret_cast<const u32x4_t *>(kt0 + (st >> 1) * 4096 + kt * 2048 +
                                                                     ((st & 1) ? koff1 : koff0)));
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                float4_t acc = (float4_t)0.0f;
#pragma unroll
                for (int st = 0; st < NS; ++st) {
                    acc = mfma(kf[st], qh[nt][st], acc);
                    acc = mfma(kf[st], ql[nt][st], acc);
                }
                sacc[kt][nt] = acc;
            }
        }
        if ((p0 < free_lo) || (p0 + 31u > free_hi)) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t key = p0 + (uint32_t)(16 * kt + 4 * g + i);
                        const bool ok      = key < ke && key >= col_lo[nt] && key <= col_hi[nt];
                        if (!ok) sacc[kt][nt][i] = -INFINITY;
                    }
        }
        /* online softmax, lazy running max (as run_segment) */
        half8_t ph[NT], pl[NT];
        float alpha_nt[NT];
        bool rose = false;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float mx = fmaxf(fmaxf(fmaxf(sacc[0][nt][0], sacc[0][nt][1]), fmaxf(sacc[0][nt][2], sacc[0][nt][3])),
                             fmaxf(fmaxf(sacc[1][nt][0], sacc[1][nt][1]), fmaxf(sacc[1][nt][2], sacc[1][nt][3])));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool raise  = mx > mrun[nt] + kLazyMax;
            const float mnew  = raise ? mx : mrun[nt];
            const float alpha = raise ? __builtin_amdgcn_exp2f(mrun[nt] - mnew) : 1.0f;
            rose             |= raise;
            alpha_nt[nt]      = alpha;
            mrun[nt]          = mnew;
            float psum        = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pv     = __builtin_amdgcn_exp2f(sacc[kt][nt][i] - mnew);
                    psum              += pv;
                    const _Float16 hi  = (_Float16)pv;
                    ph[nt][4 * kt + i] = hi;
                    if constexpr (PSPLIT) pl[nt][4 * kt + i] = (_Float16)(pv - (float)hi);
                }
            lrun[nt] = lrun[nt] * alpha + psum;
        }
        if (__builtin_amdgcn_ballot_w64(rose) != 0ull) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] *= alpha_nt[nt];
        }
        /* O^T += V^T . P^T */
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) {
            const uint8_t *vh = vt0 + (mt >> 2) * 4096; /* 64-dim half */
            const uint32_t o  = vtr ^ (32u * (uint32_t)(mt & 3));
            const half4v_t lo = lds_read_tr(vh + o);
            const half4v_t hi = lds_read_tr(vh + 16u * 128u + o);
            const half8_t av  = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                oacc[mt][nt] = mfma(av, ph[nt], oacc[mt][nt]);
                if constexpr (PSPLIT) oacc[mt][nt] = mfma(av, pl[nt], oacc[mt][nt]);
            }
        }
    }

    /* ---- epilogue (as run_segment) ------------------------------------------ */
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        float lt = lrun[nt] + __shfl_xor(lrun[nt], 16);
        lt += __shfl_xor(lt, 32);
        const uint32_t n = (uint32_t)(l16 + 16 * nt);
        if (n >= P.ncols) continue;
        const uint32_t r = n / P.kv_mul;
        const uint32_t h = kvh * P.kv_mul + (n - r * P.kv_mul);
        if (direct) {
            const size_t orow = ((size_t)s * P.n_rows + r) * P.n_head_q + h;
            const float gv    = gate_value(P.gate, orow, P.gate_is_logit);
            const float inv   = (lt > 0.0f) ? gv / lt : 0.0f;
            float *op         = P.out + orow * HD;
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const uint32_t d = (uint32_t)(16 * mt + 4 * g);
                if (d < P.out_dims)
                    *reinterpret_cast<float4 *>(op + d) = make_float4(oacc[mt][nt][0] * inv, oacc[mt][nt][1] * inv,
                                                                      oacc[mt][nt][2] * inv, oacc[mt][nt][3] * inv);
            }
        } else {
            float *po = P.part_o + (part + n) * HD;
#pragma unroll
            for (int mt = 0; mt < NM; ++mt)
                *reinterpret_cast<float4 *>(po + 16 * mt + 4 * g) =
                    make_float4(oacc[mt][nt][0], oacc[mt][nt][1], oacc[mt][nt][2], oacc[mt][nt][3]);
            if (g == 0) P.part_ml[part + n] = make_float2(mrun[nt], lt);
        }
    }
}

/* Dynamic LDS of the fused kernels: per wave, the staged new rows
 * ([n_rows][HD] K, then V, fp16). */
extern __shared__ __attribute__((aligned(16))) uint16_t fresh_lds[];

template <int HD, bool FUSE>
__device__ __forceinline__ uint16_t *fresh_area(const SplitParams &P, uint32_t wave) {
    return FUSE ? fresh_lds + (size_t)wave * 2u * P.n_rows * HD : nullptr;
}

/* Dynamic LDS bytes of a fused launch of W waves. */
template <int HD, bool FUSE>
constexpr size_t fresh_bytes(uint32_t W, uint32_t n_rows) {
    return FUSE ? (size_t)W * 2u * n_rows * HD * sizeof(uint16_t) : 0u;
}

/* Grid form: workgroup (split, head group, sequence); the W waves take W
 * adjacent KV heads over the same key chunk, so each workgroup streams
 * contiguous runs of the cache rows.  Fixed-length chunks; a sequence longer
 * than n_splits chunks gets longer chunks; splits past a short sequence's end
 * mark their partials empty. */
template <int HD, int NT, int W, bool FUSE>
__global__ __launch_bounds__(64 * W) void k_splitkv(const SplitParams P) {
    __shared__ __attribute__((aligned(16))) uint16_t vt_all[W][vt_halfs<HD>()];
    const int lane       = threadIdx.x & 63;
    const uint32_t wave  = threadIdx.x >> 6;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y * W + wave, s = blockIdx.z;
    if (kvh >= P.n_head_kv) return; /* waves only synchronise with themselves */
    const SeqKeys k      = seq_keys(P, s);
    const uint32_t total = k.last - k.lo + 1u;
    uint32_t chunk       = P.chunk;
    if ((uint64_t)chunk * P.n_splits < total) chunk = (((total + P.n_splits - 1u) / P.n_splits) + 31u) & ~31u;
    const uint32_t kb = k.lo + split * chunk;
    const uint32_t ke = min(kb + chunk, k.last + 1u); /* exclusive; empty if kb > last */
    const size_t part = ((size_t)(s * P.n_head_kv + kvh) * P.n_splits + split) * P.ncols;
    if (kb > k.last) {
        for (uint32_t n = lane; n < P.ncols; n += 64) P.part_ml[part + n] = make_float2(kNegBig, 0.0f);
        return;
    }
    run_segment<HD, NT, FUSE>(P, vt_all[wave], fresh_area<HD, FUSE>(P, wave), s, k.pos0, kvh, kb, ke,
                              P.n_splits == 1u, part);
}

/* Small batches (few (sequence, KV head) pairs): one workgroup per pair, its
 * WW waves taking the key splits, and the log-sum-exp merge done by the same
 * workgroup after a barrier, so no second kernel is launched.  The partials
 * go through the workspace as on the grid (they stay in the CU's caches). */
template <int HD, int NT, int WW, bool FUSE>
__global__ __launch_bounds__(64 * WW) void k_splitkv_wg(const SplitParams P) {
    constexpr uint32_t D4 = HD / 4;
    __shared__ __attribute__((aligned(16))) uint16_t vt_all[WW][vt_halfs<HD>()];
    const int lane       = threadIdx.x & 63;
    const uint32_t split = threadIdx.x >> 6, kvh = blockIdx.x, s = blockIdx.y;
    const SeqKeys k      = seq_keys(P, s);
    const uint32_t total = k.last - k.lo + 1u;
    uint32_t chunk       = P.chunk;
    if ((uint64_t)chunk * P.n_splits < total) chunk = (((total + P.n_splits - 1u) / P.n_splits) + 31u) & ~31u;
    const size_t base = (size_t)(s * P.n_head_kv + kvh) * P.n_splits * P.ncols;
    /* the gate of this thread's first merge item, loaded before the splits */
    float graw0 = 1.0f;
    if (threadIdx.x < P.ncols * D4) {
        const uint32_t n0 = threadIdx.x / D4, r0 = n0 / P.kv_mul;
        graw0 = gate_raw(P.gate, ((size_t)s * P.n_rows + r0) * P.n_head_q + kvh * P.kv_mul + (n0 - r0 * P.kv_mul));
    }
    if (split < P.n_splits) {
        const uint32_t kb = k.lo + split * chunk;
        const uint32_t ke = min(kb + chunk, k.last + 1u);
        const size_t part = base + (size_t)split * P.ncols;
        if (kb > k.last) {
            for (uint32_t n = (uint32_t)lane; n < P.ncols; n += 64u) P.part_ml[part + n] = make_float2(kNegBig, 0.0f);
        } else {
            run_segment<HD, NT, FUSE>(P, vt_all[split], fresh_area<HD, FUSE>(P, split), s, k.pos0, kvh, kb, ke,
                                      false, part);
        }
    }
    __syncthreads();
    for (uint32_t it = threadIdx.x; it < P.ncols * D4; it += 64u * WW) {
        const uint32_t n = it / D4, d4 = it - n * D4;
        float M = kNegBig, L = 0.0f;
        float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
        for (uint32_t sp = 0; sp < P.n_splits; ++sp) {
            const size_t idx = base + (size_t)sp * P.ncols + n;
            const float2 ml  = P.part_ml[idx];
            const float4 o   = *reinterpret_cast<const float4 *>(P.part_o + idx * HD + 4 * d4);
            if (ml.y > 0.0f) {
                const float Mn = fmaxf(M, ml.x);
                const float a  = __builtin_amdgcn_exp2f(M - Mn);
                const float b  = __builtin_amdgcn_exp2f(ml.x - Mn);
                L   = L * a + ml.y * b;
                O.x = O.x * a + o.x * b;
                O.y = O.y * a + o.y * b;
                O.z = O.z * a + o.z * b;
                O.w = O.w * a + o.w * b;
                M   = Mn;
            }
        }
        const uint32_t r  = n / P.kv_mul;
        const uint32_t h  = kvh * P.kv_mul + (n - r * P.kv_mul);
        const size_t orow = ((size_t)s * P.n_rows + r) * P.n_head_q + h;
        const float gv    = gate_apply(it == threadIdx.x ? graw0 : gate_raw(P.gate, orow), P.gate, P.gate_is_logit);
        const float inv   = (L > 0.0f) ? gv / L : 0.0f;
        const uint32_t d  = 4 * d4;
        if (d < P.out_dims)
            *reinterpret_cast<float4 *>(P.out + orow * HD + d) = make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
    }
}

/* ---- balanced plan -----------------------------------------------------------------
 * The batch's keys are cut into 32-key tiles and laid out as one sequence:
 * sequence major, then KV-head group, then tile (so the groups of a cache row
 * are read at the same time).  Workgroup g of G takes tiles
 * [g*N/G, (g+1)*N/G) of the N, split at (sequence, group) boundaries into
 * segments: every workgroup gets the same number of tiles (+-1) whatever the
 * sequence lengths, and consecutive workgroups -- which the dispatcher
 * spreads round-robin over the XCDs -- take consecutive tiles.  (A fixed
 * (split, sequence) grid puts every sequence's split k on the same XCD, so
 * short sequences leave XCDs idle.)  G is the resident workgroup count, or
 * fewer so that each takes >= min_tiles; when every sequence has the same
 * length, G is a multiple of the (sequence, group) count so that segments
 * never straddle two sequences.  The index math (shares, segments, partial
 * slots, the merge's slot range) is splitkv_plan.h, which the tests run on
 * the CPU over random ragged batches. */
__device__ __forceinline__ uint32_t wave_sum(uint32_t x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    return x;
}

struct TilePlan {
    uint32_t T;        /* tiles of all sequences, one group                   */
    uint32_t G;        /* workgroups taking part                              */
    uint32_t lane_pos; /* position of sequence `lane` (sequences 0..63)       */
    bool uniform;      /* every sequence has the same number of tiles         */
};

/* All lanes of the wave take part (wave-wide reductions). */
__device__ __forceinline__ TilePlan tile_plan(const SplitParams &P, int lane) {
    TilePlan p;
    const lfm_bal_cfg &c = P.plan;
    if (!P.pos0_dev) {
        p.lane_pos = P.pos0_host;
        p.T        = c.n_seq * lfm_bal_seq_tiles(&c, P.pos0_host);
        p.uniform  = true;
    } else {
        uint32_t sum = 0, odd = 0, t0 = 0;
        for (uint32_t b = 0; b < c.n_seq; b += 64u) {
            const uint32_t s   = b + (uint32_t)lane;
            const uint32_t pos = s < c.n_seq ? P.pos0_dev[s] : 0u;
            uint32_t x         = s < c.n_seq ? lfm_bal_seq_tiles(&c, pos) : 0u;
            if (b == 0u) {
                p.lane_pos = pos;
                t0         = __shfl(x, 0);
            }
            sum += wave_sum(x);
            if (s >= c.n_seq) x = t0;
            odd |= (uint32_t)(__ballot(x != t0) != 0);
        }
        p.T       = sum;
        p.uniform = odd == 0u;
    }
    p.G = lfm_bal_plan_wgs(&c, p.T, p.uniform);
    return p;
}

__device__ __forceinline__ uint32_t pos_of(const SplitParams &P, const TilePlan &p, uint32_t s) {
    if (!P.pos0_dev) return P.pos0_host;
    return s < 64u ? (uint32_t)__shfl(p.lane_pos, (int)s) : P.pos0_dev[s];
}

/* Ragged batches: the sequence holding tile t (0 <= t < N) and its first
 * tile -- the wave-parallel form of a prefix walk over n_groups * tiles(s). */
__device__ __forceinline__ void find_seq(const SplitParams &P, uint64_t t, int lane, uint32_t *s_out,
                                         uint64_t *first_out) {
    const lfm_bal_cfg &c = P.plan;
    uint64_t base = 0;
    for (uint32_t b = 0;; b += 64u) {
        const uint32_t s    = b + (uint32_t)lane;
        const uint32_t x    = s < c.n_seq ? lfm_bal_seq_tiles(&c, P.pos0_dev[s]) * c.n_groups : 0u;
        const uint32_t incl = wave_incl_scan(x, lane);
        const uint32_t tot  = __shfl(incl, 63);
        if (t < base + tot || b + 64u >= c.n_seq) {
            const uint64_t m = __ballot(base + incl > t);
            const int l      = m ? (int)__builtin_ctzll(m) : 0;
            *s_out           = b + (uint32_t)l;
            *first_out       = base + __shfl(incl - x, l);
            return;
        }
        base += tot;
    }
}

/* DMA: the waves run LDS-streamed segments (run_segment_dma; no fused
 * prologue), each with its DMA_NBUF-slot ring. */
template <int HD, int NT, int W, bool FUSE, bool DMA = false>
__global__ __launch_bounds__(64 * W) void k_splitkv_bal(const SplitParams P) {
    static_assert(!DMA || !FUSE, "LDS-streamed segments: no fused prologue");
    constexpr size_t LDS_BYTES = DMA ? (size_t)W * DMA_NBUF * dma_tile<HD>() : (size_t)W * vt_halfs<HD>() * 2u;
    static_assert(LDS_BYTES <= 163840, "one workgroup's LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t lds_area[LDS_BYTES];
    const lfm_bal_cfg &c = P.plan;
    const int lane       = threadIdx.x & 63;
    const uint32_t wave  = threadIdx.x >> 6;
    const uint32_t wg    = blockIdx.x;
    const TilePlan pl    = tile_plan(P, lane);
    if (wg == 0u && wave == 0u && P.pos0_dev) {
        /* tiles before each sequence and the plan, for the merge */
        uint32_t base = 0;
        for (uint32_t b = 0; b < c.n_seq; b += 64u) {
            const uint32_t s    = b + (uint32_t)lane;
            const uint32_t x    = s < c.n_seq ? lfm_bal_seq_tiles(&c, pos_of(P, pl, s)) : 0u;
            const uint32_t incl = wave_incl_scan(x, lane);
            if (s < c.n_seq) P.tile_prefix[s] = base + incl - x;
            base += __shfl(incl, 63);
        }
        if (lane == 0) {
            P.tile_prefix[c.n_seq]      = base;
            P.tile_prefix[c.n_seq + 1u] = pl.G;
        }
    }
    if (wg >= pl.G) return;
    /* One walk for both plans, so the kernel holds one copy of the segment
     * code: a uniform batch has one segment per workgroup (unit = (sequence,
     * group), n workgroups per unit, equal shares), a ragged one cuts its
     * tile share at unit boundaries. */
    lfm_bal_useg u{};
    uint64_t t = 0, t1 = 1, first = 0;
    uint32_t s = 0;
    if (pl.uniform) {
        u = lfm_bal_uniform_segment(&c, wg, pl.G, pl.T / c.n_seq);
    } else {
        lfm_bal_wg_tiles(wg, (uint64_t)pl.T * c.n_groups, pl.G, &t, &t1);
        find_seq(P, t, lane, &s, &first);
    }
    while (t < t1) {
        uint32_t seq, grp, a, b, pos0;
        uint64_t slot;
        bool direct;
        if (pl.uniform) {
            seq = u.s, grp = u.grp, a = u.a, b = u.b, slot = u.slot, direct = u.n == 1u;
            pos0 = pos_of(P, pl, seq);
            t    = t1;
        } else {
            seq                  = s;
            pos0                 = pos_of(P, pl, s);
            const uint32_t tiles = lfm_bal_seq_tiles(&c, pos0);
            const lfm_bal_seg sg = lfm_bal_segment(t, t1, first, tiles);
            grp = sg.grp, a = sg.a, b = sg.b, direct = sg.whole != 0;
            slot = lfm_bal_slot(wg, s, c.n_groups, sg.grp);
            t    = sg.end;
            if (t == first + (uint64_t)tiles * c.n_groups) {
                first = t;
                ++s;
            }
        }
        const uint32_t kvh = grp * W + wave;
        if (kvh < P.n_head_kv) {
            uint32_t kb, ke;
            lfm_bal_seg_keys(&c, pos0, a, b, &kb, &ke);
            const size_t part = ((size_t)slot * P.n_head_kv + kvh) * P.ncols;
            if constexpr (DMA)
                run_segment_dma<HD, NT>(P, lds_area + (size_t)wave * DMA_NBUF * dma_tile<HD>(), seq, pos0, kvh, kb, ke, direct,
                                    part);
            else
                run_segment<HD, NT, FUSE>(P, reinterpret_cast<uint16_t *>(lds_area) + (size_t)wave * vt_halfs<HD>(),
                                          fresh_area<HD, FUSE>(P, wave), seq, pos0, kvh, kb, ke, direct, part);
        }
    }
}

/* Merge for the balanced plan.  Four adjacent lanes share one (sequence, KV
 * head, column, 4 output dims) item: lane q of the four combines slots
 * q, q+4, ... of the workgroups that met the unit, then the four results are
 * combined through lane shuffles. */
template <int HD>
__global__ __launch_bounds__(256) void k_merge_bal(const SplitParams P) {
    constexpr uint32_t D4 = HD / 4;
    constexpr uint32_t SG = 4;
    const lfm_bal_cfg &c  = P.plan;
    const uint32_t t      = blockIdx.x * 256u + threadIdx.x;
    const uint32_t q      = t % SG;
    const uint32_t per    = P.ncols * D4; /* items per (sequence, KV head) */
    const uint32_t item   = t / SG;
    const uint32_t w      = item / per;   /* s * n_head_kv + kvh */
    const bool live       = w < c.n_seq * P.n_head_kv;
    const uint32_t wl     = live ? w : 0u;
    const uint32_t s = wl / P.n_head_kv, kvh = wl - s * P.n_head_kv;
    const uint32_t grp = kvh / P.wpg;
    const uint32_t rem = item - w * per;
    const uint32_t n = rem / D4, d4 = rem - n * D4;
    const uint32_t r  = n / P.kv_mul;
    const uint32_t h  = kvh * P.kv_mul + (n - r * P.kv_mul);
    const size_t orow = ((size_t)s * P.n_rows + r) * P.n_head_q + h;
    const float graw  = live && q == 0u ? gate_raw(P.gate, orow) : 1.0f; /* before the slot loads */
    uint32_t T, G, tiles, before;
    if (!P.pos0_dev) {
        tiles  = lfm_bal_seq_tiles(&c, P.pos0_host);
        T      = c.n_seq * tiles;
        before = s * tiles;
        G      = lfm_bal_plan_wgs(&c, T, 1);
    } else { /* the attention kernel's plan */
        before = P.tile_prefix[s];
        tiles  = P.tile_prefix[s + 1u] - before;
        T      = P.tile_prefix[c.n_seq];
        G      = P.tile_prefix[c.n_seq + 1u];
    }
    uint32_t g0, g1;
    lfm_bal_merge_range(before, tiles, grp, T, c.n_groups, G, &g0, &g1);
    float M = kNegBig, L = 0.0f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live && g0 != g1) {
        /* up to MS slots' loads per lane in flight before any is combined:
         * units of up to 16 workgroups (SG x MS) take one round trip */
        constexpr uint32_t MS = 4;
        for (uint32_t g = g0 + q; g <= g1; g += MS * SG) {
            float2 ml[MS];
            float4 o[MS];
#pragma unroll
            for (uint32_t j = 0; j < MS; ++j) {
                ml[j] = make_float2(kNegBig, 0.0f);
                o[j]  = make_float4(0.f, 0.f, 0.f, 0.f);
                if (g + j * SG <= g1) {
                    const size_t slot = (size_t)lfm_bal_slot(g + j * SG, s, c.n_groups, grp);
                    const size_t idx  = (slot * P.n_head_kv + kvh) * P.ncols + n;
                    ml[j]             = P.part_ml[idx];
                    o[j]              = *reinterpret_cast<const float4 *>(P.part_o + idx * HD + 4 * d4);
                }
            }
#pragma unroll
            for (uint32_t j = 0; j < MS; ++j) {
                if (!(ml[j].y > 0.0f)) continue;
                const float Mn = fmaxf(M, ml[j].x);
                const float a  = __builtin_amdgcn_exp2f(M - Mn);
                const float b  = __builtin_amdgcn_exp2f(ml[j].x - Mn);
                L   = L * a + ml[j].y * b;
                O.x = O.x * a + o[j].x * b;
                O.y = O.y * a + o[j].y * b;
                O.z = O.z * a + o[j].z * b;
                O.w = O.w * a + o[j].w * b;
                M   = Mn;
            }
        }
    }
    for (uint32_t off = 1; off < SG; off <<= 1) {
        const float M2 = __shfl_xor(M, (int)off), L2 = __shfl_xor(L, (int)off);
        const float x2 = __shfl_xor(O.x, (int)off), y2 = __shfl_xor(O.y, (int)off);
        const float z2 = __shfl_xor(O.z, (int)off), w2 = __shfl_xor(O.w, (int)off);
        const float Mn = fmaxf(M, M2);
        const float a  = __builtin_amdgcn_exp2f(M - Mn), b = __builtin_amdgcn_exp2f(M2 - Mn);
        L   = L * a + L2 * b;
        O.x = O.x * a + x2 * b;
        O.y = O.y * a + y2 * b;
        O.z = O.z * a + z2 * b;
        O.w = O.w * a + w2 * b;
        M   = Mn;
    }
    if (!live || g0 == g1 || q != 0u) return; /* g0 == g1: written directly */
    const float gv    = gate_apply(graw, P.gate, P.gate_is_logit);
    const float inv   = (L > 0.0f) ? gv / L : 0.0f;
    const uint32_t d  = 4 * d4;
    if (d < P.out_dims)
        *reinterpret_cast<float4 *>(P.out + orow * HD + d) = make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
}

/* Log-sum-exp merge of the key splits; applies 1/l and the gate.
 * SG adjacent lanes share one (pair, column, 4 output dims): each reduces the
 * splits sg, sg+SG, ... with a running max, then the SG partial results are
 * combined through lane shuffles and lane sg == 0 writes the output. */
template <int HD>
__global__ __launch_bounds__(256) void k_merge(const SplitParams P, uint32_t n_items, uint32_t SG) {
    constexpr uint32_t D4 = HD / 4;
    const uint32_t t    = blockIdx.x * 256u + threadIdx.x;
    const uint32_t sg   = t % SG;
    const uint32_t item = t / SG;
    const bool live     = item < n_items;
    const uint32_t d4   = item % D4;
    const uint32_t rest = item / D4;
    const uint32_t n    = rest % P.ncols;
    const uint32_t pair = live ? rest / P.ncols : 0u; /* s * n_head_kv + kvh */
    const size_t base   = (size_t)pair * P.n_splits * P.ncols + n;
    const uint32_t s  = pair / P.n_head_kv, kvh = pair % P.n_head_kv;
    const uint32_t r  = n / P.kv_mul;
    const uint32_t h  = kvh * P.kv_mul + (n - r * P.kv_mul);
    const size_t orow = ((size_t)s * P.n_rows + r) * P.n_head_q + h;
    const float graw  = live && sg == 0u ? gate_raw(P.gate, orow) : 1.0f; /* before the split loads */
    float M = kNegBig, L = 0.0f;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) {
#pragma unroll 4
        for (uint32_t sp = sg; sp < P.n_splits; sp += SG) {
            const size_t idx = base + (size_t)sp * P.ncols;
            const float2 ml  = P.part_ml[idx];
            const float4 o   = *reinterpret_cast<const float4 *>(P.part_o + idx * HD + 4 * d4);
            if (ml.y > 0.0f) {
                const float Mn = fmaxf(M, ml.x);
                const float a  = __builtin_amdgcn_exp2f(M - Mn);
                const float b  = __builtin_amdgcn_exp2f(ml.x - Mn);
                L   = L * a + ml.y * b;
                O.x = O.x * a + o.x * b;
                O.y = O.y * a + o.y * b;
                O.z = O.z * a + o.z * b;
                O.w = O.w * a + o.w * b;
                M   = Mn;
            }
        }
    }
    for (uint32_t off = 1; off < SG; off <<= 1) {
        const float M2 = __shfl_xor(M, (int)off), L2 = __shfl_xor(L, (int)off);
        const float x2 = __shfl_xor(O.x, (int)off), y2 = __shfl_xor(O.y, (int)off);
        const float z2 = __shfl_xor(O.z, (int)off), w2 = __shfl_xor(O.w, (int)off);
        const float Mn = fmaxf(M, M2);
        const float a  = __builtin_amdgcn_exp2f(M - Mn), b = __builtin_amdgcn_exp2f(M2 - Mn);
        L   = L * a + L2 * b;
        O.x = O.x * a + x2 * b;
        O.y = O.y * a + y2 * b;
        O.z = O.z * a + z2 * b;
        O.w = O.w * a + w2 * b;
        M   = Mn;
    }
    if (!live || sg != 0u) return;
    const float gv    = gate_apply(graw, P.gate, P.gate_is_logit);
    const float inv   = (L > 0.0f) ? gv / L : 0.0f;
    const uint32_t d  = 4 * d4;
    if (d < P.out_dims)
        *reinterpret_cast<float4 *>(P.out + orow * HD + d) = make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
}

template <int HD, int NT, int W, bool FUSE>
hipError_t launch_hd_nt_w(const SplitParams &p, uint32_t n_seq, hipStream_t stream) {
    dim3 grid(p.n_splits, (p.n_head_kv + W - 1) / W, n_seq);
    hipEvent_t ev0, ev1;
    profile_events(&ev0, &ev1);
    if (ev0) (void)hipEventRecord(ev0, stream);
    hipLaunchKernelGGL((k_splitkv<HD, NT, W, FUSE>), grid, dim3(64 * W), (fresh_bytes<HD, FUSE>(W, p.n_rows)), stream,
                       p);
    hipError_t e = hipGetLastError();
    if (ev1) (void)hipEventRecord(ev1, stream);
    if (e != hipSuccess || p.n_splits == 1u) return e;
    const uint32_t n_items = n_seq * p.n_head_kv * p.ncols * (HD / 4);
    uint32_t sg = 1;
    /* 2-3 splits per lane: measured on MI355X, 8 splits merge 2.2 us faster
     * with 4 lanes per output than with 2 (each lane's loads are serial) */
    while (sg < 16u && sg * 3u < p.n_splits) sg <<= 1;
    const uint64_t threads = (uint64_t)n_items * sg;
    hipLaunchKernelGGL((k_merge<HD>), dim3((uint32_t)((threads + 255u) / 256u)), dim3(256), 0, stream, p,
                       n_items, sg);
    return hipGetLastError();
}

/* ---- host side: device facts, overrides, plan choice, launches ------------ */

constexpr int kMaxDevices = 64;

/* Compute units of the current device, queried once per device. */
std::atomic<uint32_t> g_cus[kMaxDevices];
uint32_t device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256u;
    uint32_t c = dev < kMaxDevices ? g_cus[dev].load(std::memory_order_relaxed) : 0u;
    if (c) return c;
    int n = 0;
    c = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) ? (uint32_t)n
                                                                                                      : 256u;
    if (dev < kMaxDevices) g_cus[dev].store(c, std::memory_order_relaxed);
    return c;
}

/* Launch-plan overrides for tests and tuning (lfm_attn_set_tuning).  The
 * environment (LFM_ATTN_PLAN, _WAVES, _CHUNK, _MINTILES, _PREFILL_CHAIN) seeds them once, at
 * the first launch or the first lfm_attn_set_tuning; launches read only
 * these values. */
std::atomic<uint32_t> g_plan{0}, g_waves{0}, g_chunk{0}, g_min_tiles{0}, g_prefill_chain{0};
std::once_flag g_tuning_once;

int plan_code(const char *name) {
    if (!name || !name[0] || !strcmp(name, "auto")) return 0;
    if (!strcmp(name, "grid")) return 'g';
    if (!strcmp(name, "balanced")) return 'b';
    if (!strcmp(name, "wg")) return 'w';
    if (!strcmp(name, "balanced-dma")) return 'd';
    return -1;
}

uint32_t env_count(const char *name) {
    const char *e = getenv(name);
    const long v  = e ? strtol(e, nullptr, 10) : 0;
    return v > 0 && v < 0x7fffffffL ? (uint32_t)v : 0u;
}

void seed_tuning() {
    const int pc = plan_code(getenv("LFM_ATTN_PLAN"));
    g_plan.store(pc > 0 ? (uint32_t)pc : 0u);
    g_waves.store(env_count("LFM_ATTN_WAVES"));
    g_chunk.store(env_count("LFM_ATTN_CHUNK"));
    g_min_tiles.store(env_count("LFM_ATTN_MINTILES"));
    g_prefill_chain.store(env_count("LFM_ATTN_PREFILL_CHAIN"));
}

/* Split partials: the caller's scratch (the allocation-free entry point) or
 * the library workspace (grown on demand). */
void *split_ws(size_t bytes, hipStream_t stream, const Scratch *sc, int *st) {
    if (!sc) return workspace(bytes, stream, st);
    if (bytes > sc->bytes) {
        *st = LFM_ATTN_E_SCRATCH;
        return nullptr;
    }
    return sc->ptr;
}

/* Waves per workgroup: W adjacent KV heads over one key chunk.  Measured on
 * MI355X: all KV heads of a row together (W = n_head_kv, up to 8) for
 * head_dim 64; W = 2 for head_dim 128, whose waves are register-heavy. */
uint32_t choose_waves(uint32_t n_head_kv, uint32_t head_dim, const Tuning &t) {
    uint32_t w = head_dim == 64u ? 8u : 2u;
    if (t.waves) w = t.waves;
    while (w > 1u && w > n_head_kv) w >>= 1;
    return w >= 8u ? 8u : (w >= 4u ? 4u : (w >= 2u ? 2u : 1u));
}

/* Dynamic LDS of a fused-prologue workgroup of w waves (its staged new K/V
 * rows) and the V tiles every workgroup holds: together within 64 KB. */
size_t fresh_bytes_rt(uint32_t head_dim, bool fuse, uint32_t w, uint32_t n_rows) {
    return fuse ? (size_t)w * 2u * n_rows * head_dim * sizeof(uint16_t) : 0u;
}
bool lds_fits(uint32_t head_dim, bool fuse, uint32_t w, uint32_t n_rows) {
    return (size_t)w * 32u * head_dim * sizeof(uint16_t) + fresh_bytes_rt(head_dim, fuse, w, n_rows) <= 65536u;
}

/* Workgroups of k_splitkv_bal<HD, NT, W, FUSE> resident on the whole
 * device at once, with `dyn` bytes of dynamic LDS each (queried once per
 * device, instantiation and LDS size). */
template <int HD, int NT, int W, bool FUSE, bool DMA>
uint32_t resident_wgs(size_t dyn) {
    static std::atomic<uint64_t> cached[kMaxDevices]; /* (dyn + 1) << 32 | workgroups */
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256u;
    const uint64_t tag = (uint64_t)(dyn + 1u) << 32;
    if (dev < kMaxDevices) {
        const uint64_t v = cached[dev].load(std::memory_order_relaxed);
        if ((v & ~0xffffffffull) == tag) return (uint32_t)v;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_splitkv_bal<HD, NT, W, FUSE, DMA>, 64 * W,
                                                     dyn) != hipSuccess)
        return 256u;
    const uint32_t n = device_cus() * (uint32_t)(per_cu > 0 ? per_cu : 1);
    if (dev < kMaxDevices) cached[dev].store(tag | n, std::memory_order_relaxed);
    return n;
}

/* Balanced plan: launch sized for the plan the device will pick, partial
 * slots and the tile prefix table in the workspace, then the merge. */
template <int HD, int NT, int W, bool FUSE, bool DMA = false>
int launch_bal(SplitParams p, uint32_t keys_hint, const Tuning &t, hipStream_t stream, const Scratch *sc) {
    const uint32_t cus = device_cus();
    lfm_bal_cfg &c     = p.plan;
    p.wpg              = W;
    c.n_groups         = (p.n_head_kv + W - 1u) / W;
    c.n_res            = resident_wgs<HD, NT, W, FUSE, DMA>(fresh_bytes<HD, FUSE>(W, p.n_rows));
    /* 8 waves per CU over a batch of equal sequences: one residency round of
     * 8-wave workgroups at head_dim 64.  Measured on MI355X against two
     * rounds (16 waves per CU), GB/s per step: B64 x 8192 6351-6473 ->
     * 6629-6765, B16 x 8192 4708-4885 -> 5106-5253, B64 x 2048 4755-5007 ->
     * 5276-5420, LFM3 B32 x 32768 d128 6317-6333 -> 6458-6489; 12 waves per
     * CU (a partial second round) was slower than either */
    c.target_waves = 8u * cus;
    /* LDS-streamed waves: one round of the resident workgroups (the ring
     * makes one per CU resident) */
    if constexpr (DMA) c.target_waves = c.n_res * (uint32_t)W;
    /* each workgroup's partials cost about one 32-key tile per 32 query
     * columns: keep >= 12 tiles per workgroup per 32 columns (measured on
     * MI355X for 8 rows x 4 heads), and >= 2 tiles */
    c.min_tiles = (12u * p.ncols + 31u) / 32u;
    /* keys_hint bounds the keys a row attends */
    uint32_t keys = keys_hint;
    if (!p.pos0_dev) keys = p.pos0_host + p.n_rows - lfm_plan_row(p.pos0_host, p.window, p.cap).t_start;
    /* ...but a batch too small for that many workgroups per tile share
     * takes shorter shares, down to about two thirds of the resident
     * workgroups (a full residency round measured no faster, and any
     * workgroup past it doubles the time): verify 8 rows x 4 heads at B8 x
     * 4104 keys 31.9 -> 24.6 us (86 -> 172 workgroups); B16, B32 unchanged */
    const uint64_t t_max = (uint64_t)c.n_seq * c.n_groups * ((keys + 31u) / 32u + 1u);
    const uint64_t fill  = t_max * 3u / (2u * (uint64_t)(c.n_res ? c.n_res : 1u));
    if (fill < c.min_tiles) c.min_tiles = (uint32_t)fill;
    if (c.min_tiles < 2u) c.min_tiles = 2u;
    if (t.min_tiles) c.min_tiles = t.min_tiles;
    if (t.chunk) {
        /* about `chunk` keys per workgroup: enough workgroups for the longest
         * sequences keys_hint allows; longer ones get more keys */
        c.min_tiles    = (t.chunk + 31u) / 32u;
        c.n_res        = 0x7fffffffu;
        c.target_waves = 0x7fffffffu;
        keys           = p.pos0_dev ? keys_hint : p.pos0_host + p.n_rows;
        if (keys == 0u) keys = p.window ? p.window + p.n_rows - 1u : 4096u;
    }
    c.n_wg                  = lfm_bal_launch_wgs(&c, keys);
    const uint64_t n_launch = c.n_wg;
    const size_t n_part  = (size_t)lfm_bal_n_slots(c.n_wg, c.n_groups, c.n_seq) * p.n_head_kv * p.ncols;
    const size_t o_bytes = (n_part * HD * sizeof(float) + 255) & ~(size_t)255;
    const size_t m_bytes = (n_part * sizeof(float2) + 255) & ~(size_t)255;
    int st   = LFM_ATTN_OK;
    char *ws = static_cast<char *>(split_ws(o_bytes + m_bytes + ((size_t)c.n_seq + 2u) * sizeof(uint32_t), stream, sc, &st));
    if (!ws) return st;
    p.part_o      = reinterpret_cast<float *>(ws);
    p.part_ml     = reinterpret_cast<float2 *>(ws + o_bytes);
    p.tile_prefix = reinterpret_cast<uint32_t *>(ws + o_bytes + m_bytes);
    hipEvent_t ev0, ev1;
    profile_events(&ev0, &ev1);
    if (ev0) (void)hipEventRecord(ev0, stream);
    hipLaunchKernelGGL((k_splitkv_bal<HD, NT, W, FUSE, DMA>), dim3((uint32_t)n_launch), dim3(64 * W),
                       (fresh_bytes<HD, FUSE>(W, p.n_rows)), stream, p);
    hipError_t e = hipGetLastError();
    if (ev1) (void)hipEventRecord(ev1, stream);
    if (e != hipSuccess) return hip_status(e);
    const uint64_t mt = (uint64_t)c.n_seq * p.n_head_kv * p.ncols * (HD / 4) * 4u;
    hipLaunchKernelGGL((k_merge_bal<HD>), dim3((uint32_t)((mt + 255u) / 256u)), dim3(256), 0, stream, p);
    return hip_status(hipGetLastError());
}

/* Waves of the in-workgroup form: 8 (4 at head_dim 128 or 64 query columns,
 * whose waves need more than the 256 registers an 8-wave workgroup leaves
 * them). */
uint32_t wg_waves(uint32_t head_dim, uint32_t nt) { return (head_dim == 64u && nt <= 2u) ? 8u : 4u; }

/* 16-column tiles of the kernel instantiation a batch runs on. */
uint32_t tiles_of(uint32_t head_dim, uint32_t ncols) {
    const uint32_t nt = (ncols + 15u) / 16u;
    return head_dim == 64u ? (nt <= 2u ? nt : 4u) : (nt <= 1u ? 1u : 2u);
}

/* Key chunk per wave (multiple of 32) and the number of chunks the grid
 * covers.  Each wave keeps one 32-key sub-tile in flight, so throughput
 * follows the number of waves; about 4096 waves over the batch measured best
 * on MI355X (two residency rounds).  Chunks stay >= 16 x the query columns so
 * the split partials remain a small fraction of the KV bytes.
 * keys_hint bounds the keys per row; the chunk override replaces the choice. */
void choose_split(const AttnBatch &b, uint32_t keys_hint, const Tuning &t, uint32_t *n_splits, uint32_t *chunk) {
    uint32_t keys = keys_hint;
    if (keys == 0u) keys = b.window ? b.window + b.n_rows - 1u : 4096u;
    if (b.window && keys > b.window + b.n_rows - 1u) keys = b.window + b.n_rows - 1u;
    const uint64_t pairs  = (uint64_t)b.n_seq * b.n_head_kv;
    const uint64_t ncols  = (uint64_t)b.n_rows * (b.n_head_q / b.n_head_kv);
    const uint64_t target = 4096; /* waves */
    uint64_t c = ((uint64_t)keys * pairs + target - 1) / target;
    if (c < 64) c = 64;
    /* many columns (speculative verify) make each split's partial results
     * large: keep a split at least 12 keys per column (measured on MI355X
     * for 8 rows x 4 heads: 384-key chunks beat 256 and 512 by 16 %) */
    if (c < 12 * ncols) c = 12 * ncols;
    if (t.chunk) c = t.chunk;
    c = (c + 31) & ~(uint64_t)31;
    uint64_t n = (keys + c - 1) / c;
    if (n > 1024) { n = 1024; c = (((keys + n - 1) / n) + 31) & ~(uint64_t)31; }
    *n_splits = (uint32_t)(n ? n : 1);
    *chunk    = (uint32_t)c;
}

/* Launches of the chosen plan, per kernel instantiation. */
template <int HD, int NT, bool FUSE>
int launch_wg(SplitParams p, uint32_t n_seq, hipStream_t stream) {
    constexpr int WW = HD == 64 && NT <= 2 ? 8 : 4;
    if (p.n_splits > (uint32_t)WW) p.n_splits = WW; /* forced: the kernel lengthens the chunks */
    hipEvent_t ev0, ev1;
    profile_events(&ev0, &ev1);
    if (ev0) (void)hipEventRecord(ev0, stream);
    hipLaunchKernelGGL((k_splitkv_wg<HD, NT, WW, FUSE>), dim3(p.n_head_kv, n_seq), dim3(64 * WW),
                       (fresh_bytes<HD, FUSE>(WW, p.n_rows)), stream, p);
    const hipError_t e = hipGetLastError();
    if (ev1) (void)hipEventRecord(ev1, stream);
    return hip_status(e);
}

template <int HD, int NT, bool FUSE>
int launch_hd_nt(const SplitParams &p, uint32_t n_seq, uint32_t keys_hint, const PlanChoice &pc, const Tuning &t,
                 hipStream_t stream, const Scratch *sc) {
    /* a grid form with split keys writes partial slots: never launch one
     * without them */
    if (pc.kind != 'b' && pc.kind != 'd' && p.n_splits > 1u && (!p.part_o || !p.part_ml)) return LFM_ATTN_E_INVALID;
    note_plan(plan_name(pc.kind));
    if (pc.kind == 'w') return launch_wg<HD, NT, FUSE>(p, n_seq, stream);
    if (pc.kind == 'd') {
        if constexpr (HD == 64 && NT <= 2 && !FUSE) return launch_bal<HD, NT, 4, FUSE, true>(p, keys_hint, t, stream, sc);
        else if constexpr (HD == 128 && NT == 1 && !FUSE)
            return launch_bal<HD, NT, 2, FUSE, true>(p, keys_hint, t, stream, sc);
        else return LFM_ATTN_E_INVALID; /* choose_plan never picks it here */
    }
    const uint32_t w = pc.waves;
    if (pc.kind == 'b') {
        if (w == 8u) return launch_bal<HD, NT, 8, FUSE>(p, keys_hint, t, stream, sc);
        if (w == 4u) return launch_bal<HD, NT, 4, FUSE>(p, keys_hint, t, stream, sc);
        if (w == 2u) return launch_bal<HD, NT, 2, FUSE>(p, keys_hint, t, stream, sc);
        return launch_bal<HD, NT, 1, FUSE>(p, keys_hint, t, stream, sc);
    }
    hipError_t e;
    if (w == 8u) e = launch_hd_nt_w<HD, NT, 8, FUSE>(p, n_seq, stream);
    else if (w == 4u) e = launch_hd_nt_w<HD, NT, 4, FUSE>(p, n_seq, stream);
    else if (w == 2u) e = launch_hd_nt_w<HD, NT, 2, FUSE>(p, n_seq, stream);
    else e = launch_hd_nt_w<HD, NT, 1, FUSE>(p, n_seq, stream);
    return hip_status(e);
}

/* Head dim and 16-column tiles of the batch -> kernel instantiation. */
template <bool FUSE>
int dispatch_nt(const SplitParams &p, const AttnBatch &b, uint32_t keys_hint, const PlanChoice &pc, const Tuning &t,
                hipStream_t stream, const Scratch *sc) {
    const uint32_t nt = tiles_of(b.head_dim, p.ncols);
    if (b.head_dim == 64u) {
        if (nt == 1u) return launch_hd_nt<64, 1, FUSE>(p, b.n_seq, keys_hint, pc, t, stream, sc);
        if (nt == 2u) return launch_hd_nt<64, 2, FUSE>(p, b.n_seq, keys_hint, pc, t, stream, sc);
        return launch_hd_nt<64, 4, FUSE>(p, b.n_seq, keys_hint, pc, t, stream, sc);
    }
    if (nt == 1u) return launch_hd_nt<128, 1, FUSE>(p, b.n_seq, keys_hint, pc, t, stream, sc);
    return launch_hd_nt<128, 2, FUSE>(p, b.n_seq, keys_hint, pc, t, stream, sc);
}

} // namespace

/* Plan choice (host only, no device access):
 *  - grid or balanced: a batch whose sequences may differ in length
 *    (positions on the device, more than one sequence) takes the balanced
 *    plan: measured on MI355X, 64 sequences of 512..8192 keys run 23 %
 *    faster than on the fixed-chunk grid, which leaves XCDs idle.  A batch
 *    that cannot be ragged (one sequence, or one shared host position) takes
 *    the grid, which skips the plan's position scan and table (1-9 % faster
 *    on equal-length batches).  So does a sliding-window batch: no row reads
 *    more than window keys, which bounds how ragged it can be (config 5's
 *    ring, B32 x 256 keys: 10.7 vs 11.9 us per call).
 *  - the grid's in-workgroup form (k_splitkv_wg: one workgroup per (sequence,
 *    KV head), the key splits as its waves, the merge inside it): for grid
 *    batches of at most as many pairs as compute units whose planned splits
 *    fit the workgroup's waves (short contexts, sliding windows), where a
 *    second (merge) launch would cost about as much as the attention itself.
 *    Measured on MI355X (us per call, grid + merge kernel -> this form): SWA
 *    window 256, d128 16q/4kv, B16 11.2 -> 10.8, B32 12.3 -> 11.2, B64 15.2
 *    -> 12.5; d64 32q/8kv, B32 11.3 -> 8.5; with more planned splits than
 *    waves (window 512: 8 splits, 4 waves) the grid stays faster (15.6 vs
 *    17.4), and lengthening the splits to fit measured slower than the
 *    second launch (B1 ctx 1024, 16 splits on 8 waves: 10.3 vs 8.5 us).
 *  - waves per workgroup (choose_waves), fewer where a fused prologue's
 *    staged rows and the V tiles would pass 64 KB of LDS, and a grid of
 *    fewer workgroups than compute units (one short sequence) spreads its KV
 *    heads over more, smaller workgroups: measured on MI355X at B1, 8 KV
 *    heads, ctx 256-4096, 9.6-12.0 us -> 8.2-10.5 us per call (8-row verify
 *    at ctx 4096: 29.2 -> 22.0 us); larger grids unchanged.
 * The overrides force a plan ('g', 'b', 'w'), waves or a chunk; a waves or
 * chunk override keeps the grid off its in-workgroup form. */
/* Batches the LDS-streamed balanced form runs: no fused prologue; head_dim
 * 64 with at most two 16-column tiles (4-wave workgroups), or head_dim 128
 * with one (2-wave workgroups: a wave's ring is 64 KB). */
static bool dma_eligible(const AttnBatch &b, bool fuse) {
    const uint32_t nt = tiles_of(b.head_dim, b.n_rows * (b.n_head_q / b.n_head_kv));
    return !fuse && ((b.head_dim == 64u && nt <= 2u) || (b.head_dim == 128u && nt == 1u));
}

PlanChoice choose_plan(const AttnBatch &b, uint32_t keys_hint, bool positions_on_device, bool fuse, uint32_t cus,
                       const Tuning &t) {
    PlanChoice pc{};
    const uint32_t ncols  = b.n_rows * (b.n_head_q / b.n_head_kv);
    bool grid             = !positions_on_device || b.n_seq == 1u || b.window != 0u;
    if (t.plan == 'g' || t.plan == 'w') grid = true;
    if (t.plan == 'b' || t.plan == 'd') grid = false;
    if (grid) {
        choose_split(b, keys_hint, t, &pc.n_splits, &pc.chunk);
        const uint32_t ww = wg_waves(b.head_dim, tiles_of(b.head_dim, ncols));
        bool wg = false;
        if (t.plan == 'w') wg = pc.n_splits >= 2u;
        else if (t.plan != 'g' && !t.waves && !t.chunk)
            wg = pc.n_splits >= 2u && pc.n_splits <= ww && (uint64_t)b.n_seq * b.n_head_kv <= cus;
        if (wg && lds_fits(b.head_dim, fuse, ww, b.n_rows)) {
            pc.kind  = 'w';
            pc.waves = ww;
            if (pc.n_splits > ww) pc.n_splits = ww;
            return pc;
        }
    }
    uint32_t w = choose_waves(b.n_head_kv, b.head_dim, t);
    while (w > 1u && !lds_fits(b.head_dim, fuse, w, b.n_rows)) w >>= 1;
    if (grid && !t.waves)
        while (w > 1u && (uint64_t)pc.n_splits * ((b.n_head_kv + w - 1u) / w) * b.n_seq < cus) w >>= 1;
    pc.kind  = grid ? 'g' : 'b';
    pc.waves = w;
    /* the LDS-streamed form: forced, or by default for two 16-column tiles
     * (speculative verify), where it measured faster on MI355X -- B16 x 8
     * rows x 4104 keys 39.9-40.1 -> 37.6-37.9 us per step -- while one-tile
     * batches run faster on the register form (B64 x 8192: 158.4-159.7 vs
     * 162.4-163.6 us; ragged B64: 98.3-98.7 vs 102.1-102.7 us) */
    const bool dma_default = t.plan == 0 && !t.waves && tiles_of(b.head_dim, ncols) == 2u;
    if (!grid && (t.plan == 'd' || dma_default) && dma_eligible(b, fuse)) {
        pc.kind  = 'd';
        pc.waves = b.head_dim == 128u ? 2u : 4u;
    }
    return pc;
}

const char *plan_name(char kind) {
    return kind == 'w' ? "wg" : kind == 'g' ? "grid" : kind == 'd' ? "balanced-dma" : "balanced";
}

Tuning current_tuning() {
    std::call_once(g_tuning_once, seed_tuning);
    return Tuning{(char)g_plan.load(), g_waves.load(), g_chunk.load(), g_min_tiles.load(), g_prefill_chain.load()};
}

int set_tuning(const char *plan, uint32_t waves, uint32_t chunk, uint32_t min_tiles, uint32_t prefill_chain) {
    const int pc = plan_code(plan);
    if (pc < 0 || (waves && waves != 1u && waves != 2u && waves != 4u && waves != 8u)) return LFM_ATTN_E_INVALID;
    std::call_once(g_tuning_once, seed_tuning);
    g_plan.store((uint32_t)pc);
    g_waves.store(waves);
    g_chunk.store(chunk);
    g_min_tiles.store(min_tiles);
    g_prefill_chain.store(prefill_chain);
    return LFM_ATTN_OK;
}

bool splitkv_supports(const AttnBatch &b) {
    if (b.head_dim != 64u && b.head_dim != 128u) return false;
    const uint32_t kv_mul = b.n_head_q / b.n_head_kv;
    const uint32_t ncols  = b.n_rows * kv_mul;
    if (b.head_dim == 64u) return ncols <= 64u;
    return ncols <= 32u;
}

int launch_splitkv(const AttnBatch &b, uint32_t keys_hint, hipStream_t stream, const Scratch *sc) {
    if (!splitkv_supports(b)) return LFM_ATTN_E_UNSUPPORTED;
    SplitParams p{};
    p.q             = b.q;
    p.gate          = b.gate;
    p.gate_is_logit = b.gate_is_logit;
    p.k_base        = static_cast<const uint16_t *>(b.k_base);
    p.v_base        = static_cast<const uint16_t *>(b.v_base);
    p.k_seq         = reinterpret_cast<const uint16_t *const *>(b.k_seq);
    p.v_seq         = reinterpret_cast<const uint16_t *const *>(b.v_seq);
    p.seq_stride    = b.seq_stride;
    p.pos0_dev      = b.pos0_dev;
    p.pos0_host     = b.pos0_host;
    p.out           = b.out;
    p.n_rows        = b.n_rows;
    p.n_head_q      = b.n_head_q;
    p.n_head_kv     = b.n_head_kv;
    p.kv_mul        = b.n_head_q / b.n_head_kv;
    p.ncols         = b.n_rows * p.kv_mul;
    p.window        = b.window;
    p.cap           = b.cap;
    p.out_dims      = b.out_dims;
    p.qscale        = b.scale * kLog2e;
    p.plan.n_seq    = b.n_seq;
    p.plan.n_rows   = b.n_rows;
    p.plan.n_head_kv = b.n_head_kv;
    p.plan.window   = b.window;
    p.plan.cap      = b.cap;
    p.k_new         = b.k_new;
    p.v_new         = b.v_new;
    p.q_norm_w      = b.q_norm_w;
    p.k_norm_w      = b.k_norm_w;
    p.cos_lut       = b.cos_lut;
    p.sin_lut       = b.sin_lut;
    p.eps           = b.eps;
    p.prologue      = b.prologue;
    const Tuning t       = current_tuning();
    const PlanChoice pc  = choose_plan(b, keys_hint, b.pos0_dev != nullptr, b.k_new != nullptr, device_cus(), t);
    p.n_splits = pc.n_splits;
    p.chunk    = pc.chunk;
    /* both grid forms keep per-split partials in the workspace (the
     * in-workgroup form merges them after a barrier); the balanced plan
     * sizes its own */
    if (pc.kind != 'b' && pc.kind != 'd' && p.n_splits > 1u) {
        const size_t n_part = (size_t)b.n_seq * b.n_head_kv * p.n_splits * p.ncols;
        const size_t bytes  = n_part * b.head_dim * sizeof(float) + n_part * sizeof(float2) + 256;
        int st              = LFM_ATTN_OK;
        char *ws            = static_cast<char *>(split_ws(bytes, stream, sc, &st));
        if (!ws) return st;
        p.part_o  = reinterpret_cast<float *>(ws);
        p.part_ml = reinterpret_cast<float2 *>(ws + ((n_part * b.head_dim * sizeof(float) + 255) & ~(size_t)255));
    }
    return b.k_new ? dispatch_nt<true>(p, b, keys_hint, pc, t, stream, sc)
                   : dispatch_nt<false>(p, b, keys_hint, pc, t, stream, sc);
}

} // namespace lfm
