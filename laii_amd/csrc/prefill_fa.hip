/*
 * prefill_fa.hip -- causal prefill attention on gfx950 MFMA (fp32 Q, fp16
 * K/V cache, fp32 softmax and accumulation, fp32 output).
 *
 * Semantics: lfm2_forward_gqa_batch (tools/lfm2_prefill_batch.c:1029-1092)
 * runs the per-head task once per query row; row i (position pos_0 + i)
 * attends keys [0, pos_0 + i] of its cache (causal by write order).  This
 * kernel computes all rows of a prompt in one launch.
 *
 * Workgroup = 4 waves = TQ query positions x kv_mul query heads of one KV
 * head (256 query columns, TQ = 256 / kv_mul), so each K/V block staged in
 * LDS serves every query head that reads it.
 *
 * Staging: 64-key K and V blocks (row-major, 128-B rows) move from global
 * memory straight into a ring of 4 LDS blocks (global_load_lds_dwordx4, no
 * registers): block b + 2 is in flight while block b is computed and block
 * b - 1 is still read by the P.V product that trails the scores by a step.
 * The 16-B chunks of row r are XOR-swizzled by r & 7, which makes both the
 * K fragment reads (ds_read_b128) and the transposing V reads
 * (ds_read_b64_tr_b16) bank-conflict free on gfx950's LDS (measured with
 * SQ_LDS_BANK_CONFLICT: zero; the earlier swizzle 2*((r >> 2) & 3), laid
 * out for half as many banks, spent half of the LDS cycles in conflicts).
 *
 * Compute runs in 32-key steps.  Step k computes S^T(k+1) into a second
 * register set, turns the scores S^T(k) into P and runs PV(k): the MFMAs of
 * S^T(k+1) overlap the exponentials of P(k) within the wave, and the two
 * waves of each SIMD overlap each other's:
 *   S^T(k+1) = K . Q^T - m   16x16x32 f16 MFMA on Q * scale * log2(e),
 *                            rounded once from fp32 to fp16, so scores come
 *                            out in log2 units; the running max enters as
 *                            the accumulator's initial value
 *   p = exp2(S^T(k))         in fp32.  Lazy max: raised only when a step
 *                            exceeds it by more than 8 (P <= 2^8, fp16 P
 *                            stays finite), which rescales O and l in a
 *                            rare uniform branch
 *   O^T += V^T . P^T(k)      V^T fragments read transposed from row-major V
 *   l += 1 . P^T(k)          one more MFMA with an all-ones A operand: the
 *                            column sums of the same fp16 P, in fp32, on
 *                            the matrix pipe (v_dot2 on the VALU cannot
 *                            co-issue with MFMA)
 * Causal masking only touches steps that cross the diagonal; steps above it
 * are skipped.  Workgroups run heaviest-first (late query tiles first).
 */
#include <hip/hip_runtime.h>

#include <type_traits>

#include "kernels.h"
#include "lfm_attn.h"

namespace lfm {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4;

constexpr float kLog2e  = 1.4426950408889634f;
constexpr int KB        = 64;          /* keys per LDS block                       */
constexpr int SB        = 32;          /* keys per compute step                    */
constexpr int NBUF      = 4;           /* LDS ring of K/V blocks                   */
constexpr int ROWB      = 128;         /* bytes per K/V row of one head (d = 64)   */
constexpr int BLKB      = KB * ROWB;   /* bytes per K (or V) block                 */
constexpr float kLazy   = 8.0f;        /* headroom in log2 units (P <= 2^8)         */

struct PrefillParams {
    const float *q;     /* [n_seq][n_tok][n_head_q][HD] fp32 */
    const uint16_t *k;  /* seq s at k + s*kv_seq_stride: [slot][n_head_kv][HD] */
    const uint16_t *v;
    float *out;         /* [n_seq][n_tok][n_head_q][HD] */
    uint64_t kv_seq_stride;
    uint32_t n_seq, n_tok, pos_0, n_head_q, n_head_kv, kv_mul, tq, n_qtiles;
    float qmul;         /* softmax scale * log2(e), applied to Q before its fp16 rounding */
};

__device__ __forceinline__ half8_t as_half8(u32x4_t v) { return __builtin_bit_cast(half8_t, v); }

__device__ __forceinline__ float4_t mfma(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

/* exp2 of two scores (log2 units) in fp32, packed to fp16 with round
 * toward zero */
__device__ __forceinline__ half2_t exp_pk(float a, float b) {
    return __builtin_bit_cast(half2_t,
                              __builtin_amdgcn_cvt_pkrtz(__builtin_amdgcn_exp2f(a), __builtin_amdgcn_exp2f(b)));
}

/* transposing LDS read: within each 16-lane group, lane l receives element
 * l % 4 of the 8-byte chunks addressed by lanes l/4, l/4 + 4, l/4 + 8 and
 * l/4 + 12 */
__device__ __forceinline__ half4_t lds_read_tr(const uint8_t *p) {
    return __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4 *)p));
}

__device__ __forceinline__ float max3(float a, float b, float c) {
    return fmaxf(fmaxf(a, b), c);
}

/* 16 B per lane from global memory into LDS: lane l writes bytes
 * [lds + 16 l, lds + 16 l + 16) of the wave's 1-KB piece at LDS address lds
 * (held in M0).  The load counts in vmcnt like any other vector load; the
 * caller waits for it explicitly before the barrier that publishes it. */
__device__ __forceinline__ void fetch16_lds(const void *gaddr, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gaddr), "{m0}"(lds) : "memory");
}
/* the same from a wave-uniform base (SGPRs) plus a 32-bit per-lane byte
 * offset: no per-lane 64-bit address arithmetic */
__device__ __forceinline__ void fetch16_lds(uint32_t voff, const void *sbase, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}

template <int HD>
__global__ __launch_bounds__(256, 2) void k_prefill(const PrefillParams P) {
    static_assert(HD == 64, "prefill kernel is specialised for head_dim 64");
    constexpr int NT = 4; /* 16-column tiles per wave (64 columns) */
    constexpr int NM = HD / 16;
    /* ring of NBUF blocks, each K (8 KB) then V (8 KB) */
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NBUF * 2 * BLKB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    /* 1-D grid, heaviest query tiles first across all (sequence, KV head)
     * pairs; consecutive workgroups take consecutive pairs, so with a pair
     * count divisible by 8 the tiles of one pair land on one XCD (round-robin
     * dispatch) and share its L2 */
    const uint32_t pairs = P.n_head_kv * P.n_seq;
    const uint32_t qt    = P.n_qtiles - 1u - blockIdx.x / pairs;
    const uint32_t pair  = blockIdx.x % pairs;
    const uint32_t kvh = pair % P.n_head_kv, s = pair / P.n_head_kv;
    const uint32_t t0  = qt * P.tq; /* first query row of the tile */

    const uint16_t *kc = P.k + (size_t)s * P.kv_seq_stride + (size_t)kvh * HD;
    const uint16_t *vc = P.v + (size_t)s * P.kv_seq_stride + (size_t)kvh * HD;
    const size_t row   = (size_t)P.n_head_kv * HD;

    const uint32_t lo_pos = P.pos_0 + t0;                               /* smallest query position */
    const uint32_t hi_pos = P.pos_0 + min(t0 + P.tq, P.n_tok) - 1u;     /* largest query position  */
    const uint32_t n_keys = hi_pos + 1u;
    const uint32_t nblk   = (n_keys + KB - 1) / KB;
    const uint32_t nsub   = (n_keys + SB - 1) / SB;
    /* steps [0, nfull) lie entirely at or below the lowest query row */
    const uint32_t nfull  = min((lo_pos + 1u) / SB, nsub);

    /* ---- staging: thread tid moves 16-B chunks tid and tid + 256 of each
     * 8-KB K and V block; chunk p sits at byte 16*p of the block (row p/8,
     * slot p%8) and holds the row's global chunk (p%8) ^ swz(row).  Wave w's
     * chunks form the 1-KB pieces w and w + 4 of the block. */
    uint32_t st_row[2], st_col[2], st_off[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t p = (uint32_t)tid + 256u * e, r = p >> 3;
        st_row[e] = r;
        st_col[e] = 8u * ((p & 7u) ^ (r & 7u));                        /* halfs */
        st_off[e] = (r * (uint32_t)row + st_col[e]) * sizeof(uint16_t); /* bytes */
    }
    const uint32_t wv       = __builtin_amdgcn_readfirstlane((uint32_t)wave);
    const uint32_t ring_lds = (uint32_t)(uintptr_t)ring; /* LDS address of the ring */
    const size_t blk_bytes  = (size_t)KB * row * sizeof(uint16_t);
    /* 4 fetches per wave and block (vmcnt counts them) */
    auto fetch_block = [&](uint32_t blk) {
        const uint32_t slot = ring_lds + (blk % NBUF) * (2 * BLKB);
        if ((blk + 1u) * KB <= n_keys) {
            /* a whole block: uniform base, fixed per-lane offsets */
            const uint8_t *kb = reinterpret_cast<const uint8_t *>(kc) + blk * blk_bytes;
            const uint8_t *vb = reinterpret_cast<const uint8_t *>(vc) + blk * blk_bytes;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t piece = slot + 1024u * (wv + 4u * (uint32_t)e);
                fetch16_lds(st_off[e], kb, piece);
                fetch16_lds(st_off[e], vb, piece + (uint32_t)BLKB);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                uint32_t key = blk * KB + st_row[e];
                key = key < n_keys ? key : n_keys - 1u; /* rows past the keys: masked */
                const size_t off     = (size_t)key * row + st_col[e];
                const uint32_t piece = slot + 1024u * (wv + 4u * (uint32_t)e);
                fetch16_lds(kc + off, piece);
                fetch16_lds(vc + off, piece + (uint32_t)BLKB);
            }
        }
    };

    /* the first two blocks are in flight before the Q loads: the wait for Q
     * (which also covers these older fetches) then takes one memory round
     * trip, not two */
    fetch_block(0u);
    if (nblk > 1u) fetch_block(1u);

    /* ---- columns of this lane: (head j, row t) per N-tile -------------- */
    uint32_t col_pos[NT]; /* absolute position of the column's query row */
    bool col_ok[NT];
    half8_t qf[NT][HD / 32];
    /* all Q loads are issued before any is used (qp is a valid row for a
     * padding column too; its values are zeroed after): with a use between
     * them the compiler waited for each column tile's loads, one memory
     * round trip per tile */
    float4 qraw[NT][HD / 32][2];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t c = (uint32_t)(wave * 64 + nt * 16 + l16);
        const uint32_t j = c / P.tq, t = t0 + c % P.tq;
        col_ok[nt]  = t < P.n_tok;
        col_pos[nt] = P.pos_0 + t;
        const float *qp = P.q + (((size_t)s * P.n_tok + (col_ok[nt] ? t : 0u)) * P.n_head_q +
                                 kvh * P.kv_mul + j) * HD + 8 * g;
#pragma unroll
        for (int st = 0; st < HD / 32; ++st) {
            qraw[nt][st][0] = *reinterpret_cast<const float4 *>(qp + 32 * st);
            qraw[nt][st][1] = *reinterpret_cast<const float4 *>(qp + 32 * st + 4);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int st = 0; st < HD / 32; ++st) {
            const float4 a = qraw[nt][st][0], b = qraw[nt][st][1];
            const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            half8_t h;
            /* one fp16 rounding of q * scale * log2(e): the score
             * accumulator holds q.k in log2 units, so the exponentials need
             * no multiply */
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = col_ok[nt] ? (_Float16)(x[e] * P.qmul) : (_Float16)0.0f;
            qf[nt][st] = h;
        }

    /* fragment offsets in a block (bytes).  K: row 16*mt + l16, chunk 4*st + g.
     * V (transposing read): lane l16 of group g addresses row 4g + l16/4 of
     * a 16-key half, dims 16*mt + 4*(l16 % 4) */
    const uint32_t kswz  = (uint32_t)(g ^ (l16 & 7));
    const uint32_t koff0 = (uint32_t)l16 * ROWB + 16u * kswz;
    const uint32_t koff1 = (uint32_t)l16 * ROWB + 16u * (kswz ^ 4u);
    const uint32_t vr    = (uint32_t)(4 * g + (l16 >> 2)); /* V row read (its + 16 twin has the same swizzle) */
    uint32_t voff[NM];
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
        voff[mt] = BLKB + vr * ROWB + 16u * ((2u * (uint32_t)mt + (uint32_t)((l16 >> 1) & 1)) ^ (vr & 7u)) +
                   8u * (l16 & 1);

    float4_t oacc[NM][NT];
    float4_t negm[NT]; /* -m splat: initial value of the score accumulator */
    float4_t lacc[NT]; /* column sums of P (every element holds the column's sum) */
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        negm[nt] = (float4_t)0.0f;
        lacc[nt] = (float4_t)0.0f;
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] = (float4_t)0.0f;
    }
    const half8_t ones8 = (half8_t)(_Float16)1.0f;

    /* S^T of step k: two 16-key tiles x NT column tiles */
    auto scores = [&](auto mask_tag, uint32_t k, float4_t (&sc)[2][NT]) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const uint8_t *kb = ring + ((k >> 1) % NBUF) * (2 * BLKB) + (k & 1u) * (SB * ROWB);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const half8_t k0 = as_half8(*reinterpret_cast<const u32x4_t *>(kb + mt * 16 * ROWB + koff0));
            const half8_t k1 = as_half8(*reinterpret_cast<const u32x4_t *>(kb + mt * 16 * ROWB + koff1));
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) sc[mt][nt] = mfma(k1, qf[nt][1], mfma(k0, qf[nt][0], negm[nt]));
        }
        if constexpr (MASK) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t key = k * SB + (uint32_t)(16 * mt + 4 * g + i);
                        if (key > col_pos[nt]) sc[mt][nt][i] = -INFINITY;
                    }
        }
    };

    /* lazy max: raise m (and rescale O, l and the pending scores) when a
     * column's step maximum exceeds it by more than kLazy; the first step
     * sets m to the exact column maximum.  step_max() is the per-lane part,
     * rescale() the rare, wave-uniform branch. */
    auto step_max = [&](auto first_tag, const float4_t (&sc)[2][NT], float (&mx)[NT]) {
        constexpr bool FIRST = decltype(first_tag)::value;
        bool any_raise = FIRST;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float v = max3(max3(sc[0][nt][0], sc[0][nt][1], sc[0][nt][2]), sc[0][nt][3], sc[1][nt][0]);
            v = max3(max3(v, sc[1][nt][1], sc[1][nt][2]), sc[1][nt][3], -INFINITY);
            mx[nt] = v;
            if constexpr (!FIRST) any_raise |= v > kLazy;
        }
        return any_raise;
    };
    auto rescale = [&](auto first_tag, bool any_raise, float4_t (&sc)[2][NT], const float (&mx)[NT]) {
        constexpr bool FIRST = decltype(first_tag)::value;
        if (__builtin_amdgcn_ballot_w64(any_raise) != 0ull) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                float v = mx[nt]; /* column max over the 4 lanes holding it */
                v = fmaxf(v, __shfl_xor(v, 16));
                v = fmaxf(v, __shfl_xor(v, 32));
                const bool raise  = FIRST ? (v > -INFINITY) : (v > kLazy);
                const float inc   = raise ? v : 0.0f;
                /* O and l are still zero at the first step: no rescale
                 * (exp2(-m) overflows to inf for m < -128, and 0 * inf is
                 * NaN) */
                const float alpha = FIRST ? 1.0f : __builtin_amdgcn_exp2f(-inc);
                negm[nt] -= inc;
                lacc[nt] *= alpha;
                sc[0][nt] -= inc;
                sc[1][nt] -= inc;
#pragma unroll
                for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] *= alpha;
            }
        }
    };

    /* P^T(k) = exp2(S^T(k)), O^T += V^T(k) . P^T(k), l += 1 . P^T(k) */
    auto accumulate = [&](uint32_t k, const float4_t (&sc)[2][NT]) {
        u32x4_t pf[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const float4_t a = sc[0][nt], c = sc[1][nt];
            /* scalar temporaries: a bit_cast of an ext-vector element was
             * miscompiled into four reads of element 0 */
            const half2_t h0 = exp_pk(a[0], a[1]);
            const half2_t h1 = exp_pk(a[2], a[3]);
            const half2_t h2 = exp_pk(c[0], c[1]);
            const half2_t h3 = exp_pk(c[2], c[3]);
            u32x4_t w;
            w[0] = __builtin_bit_cast(uint32_t, h0);
            w[1] = __builtin_bit_cast(uint32_t, h1);
            w[2] = __builtin_bit_cast(uint32_t, h2);
            w[3] = __builtin_bit_cast(uint32_t, h3);
            pf[nt] = w;
        }
        const uint8_t *vb = ring + ((k >> 1) % NBUF) * (2 * BLKB) + (k & 1u) * (SB * ROWB);
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) {
            const half4_t lo = lds_read_tr(vb + voff[mt]);
            const half4_t hi = lds_read_tr(vb + 16 * ROWB + voff[mt]);
            const half8_t av = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) oacc[mt][nt] = mfma(av, as_half8(pf[nt]), oacc[mt][nt]);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) lacc[nt] = mfma(ones8, as_half8(pf[nt]), lacc[nt]);
    };

    /* entering LDS block b (at the start of step 2b - 1, before S^T(2b)):
     * this wave's fetches of block b have landed (those of block b + 1 may
     * still be in flight), and the barrier makes every wave's part visible.
     * Block b - 1 is still in use (P.V of step 2b - 1); the slot of block
     * b + 2 held block b - 2, which every wave finished before the barrier,
     * so block b + 2 is fetched into it. */
    auto enter_block = [&](uint32_t b) {
        if (b + 1u < nblk) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (b + 2u < nblk) fetch_block(b + 2u);
    };

    /* ---- steps: P(k) and PV(k), then S^T(k + 1) in the same registers -- */
    enter_block(0u);
    float4_t scur[2][NT];
    if (nfull > 0u) scores(std::false_type{}, 0u, scur);
    else scores(std::true_type{}, 0u, scur);
    {
        float mx[NT];
        const bool any_raise = step_max(std::true_type{}, scur, mx);
        rescale(std::true_type{}, any_raise, scur, mx);
    }

    /* Step k computes S^T(k + 1) into the other register set before P(k), so
     * its MFMAs overlap the exponentials of P(k) within the wave; the loop
     * runs two steps per iteration with the sets swapping roles (no register
     * copies).  Measured on MI355X at B4 x 4096 against computing S^T(k + 1)
     * after P(k) in the same registers: 127.7 vs 137.3 k cycles per
     * workgroup, bit-identical (253 VGPRs, no spills). */
    float4_t snxt[2][NT];
    auto step = [&](auto mask_tag, uint32_t k, float4_t(&sc)[2][NT], float4_t(&sn)[2][NT])
                    __attribute__((always_inline)) {
        if (((k + 1u) & 1u) == 0u) enter_block((k + 1u) >> 1);
        /* raised issue priority over the MFMA phases (S^T(k + 1), then P(k),
         * P.V and the row sums): the wave about to feed the matrix pipe wins
         * the arbiter over its SIMD partner, whose max test, rescale and
         * barrier fill the gaps.  Measured on MI355X at B4 x 4096 (N(0,1)
         * data, same process, interleaved): 264.1-269.1 vs 269.0-280.0 us;
         * the priority around the scores alone, or around P.V alone, or
         * held through the max test, measured no faster. */
        __builtin_amdgcn_s_setprio(1);
        scores(mask_tag, k + 1u, sn);
        accumulate(k, sc);
        __builtin_amdgcn_s_setprio(0);
        float mx[NT];
        const bool any_raise = step_max(std::false_type{}, sn, mx);
        rescale(std::false_type{}, any_raise, sn, mx);
    };
    uint32_t k = 0;
    /* steps k .. k_end - 1; S^T(k) is in scur on entry and on exit */
    auto run_steps = [&](auto mask_tag, uint32_t k_end) __attribute__((always_inline)) {
        for (; k + 2u <= k_end; k += 2u) {
            step(mask_tag, k, scur, snxt);
            step(mask_tag, k + 1u, snxt, scur);
        }
        if (k < k_end) {
            step(mask_tag, k, scur, snxt);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) scur[mt][nt] = snxt[mt][nt];
            ++k;
        }
    };
    run_steps(std::false_type{}, nfull > 0u ? nfull - 1u : 0u); /* S^T(k + 1) unmasked */
    run_steps(std::true_type{}, nsub - 1u);
    accumulate(k, scur);

    /* ---- epilogue: O / l ------------------------------------------------- */
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float lt = lacc[nt][0];
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

int launch_prefill(const float *q, const uint16_t *k, const uint16_t *v, float *out,
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
    P.qmul = scale * kLog2e;
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
