/*
 * prefill_ext.hip -- causal prefill on gfx950 MFMA for head_dim 128 (the LFM3
 * full and sliding-window layers), with an optional sliding window and the
 * sigmoid output gate (fp32 Q, fp16 K/V, fp32 softmax and accumulation, fp32
 * output).
 *
 * Semantics: lfm3_forward_batch_core (tools/lfm3_engine.c:1918-2055) runs
 * the attention of every prompt row over [t_start(pos), pos] of its layer's
 * cache -- t_start = pos + 1 - window for a sliding window, 0 otherwise
 * (:862-873) -- and scales the result by sigmoid(gate) (:1983-2004,
 * :902-911).  Here every row of a prompt runs in one launch.  K/V row r of
 * the buffer holds position kv_pos0 + r, so a full layer passes its cache
 * (kv_pos0 = 0) and a sliding-window layer a linear staging copy of the
 * window before the prompt plus the prompt's rows.
 *
 * Workgroup = 4 waves = 128 query columns: TQ = 128 / kv_mul positions x
 * kv_mul query heads of one KV head, so each K/V block staged in LDS serves
 * every query head that reads it; 32 columns per wave.
 *
 * Each 32-key block of K (and of V) is kept in LDS as two 64-dim halves of
 * [32 keys][128 B], with the 16-B chunks of row r XOR-swizzled by
 * r & 7: the layout of the head_dim-64 prefill kernel
 * (prefill_fa.hip), whose K fragment reads (ds_read_b128) and transposing V
 * reads (ds_read_b64_tr_b16) it serves without bank conflicts.  Blocks move
 * from global memory straight into a ring of 4 LDS blocks
 * (global_load_lds_dwordx4): block b + 2 is in flight while S^T(b) is
 * computed and block b - 1 is still read by P.V; one barrier per block.
 *
 * Per 32-key block (software pipelined as in the head_dim-64 kernel: step b
 * computes S^T(b + 1) into a second register set, then P(b) and PV(b), so
 * the MFMAs of the scores overlap the exponentials within the wave):
 *   S^T = K . Q^T - m        16x16x32 f16 MFMA on q * scale * log2(e)
 *                            rounded once to fp16 (scores in log2 units);
 *                            the running max is the accumulator's initial
 *                            value
 *   p = exp2(S^T)            lazy max: raised only when a block exceeds it
 *                            by more than 8 (P <= 2^8)
 *   O^T += V^T . P^T, l += 1 . P^T   (row sums of the same fp16 P on the
 *                            matrix pipe)
 * Blocks below the lowest row's window and above the highest row are
 * skipped; only blocks crossing the diagonal or the window's lower edge are
 * masked.  Workgroups run heaviest-first, except that a sliding-window
 * launch starts with the tiles whose window the sequence start cuts short.
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

constexpr float kLog2e = 1.4426950408889634f;
constexpr int KB       = 32;            /* keys per block (one compute step)       */
constexpr int NBUF     = 4;             /* LDS ring of blocks                      */
constexpr int HALFB    = KB * 128;      /* bytes of one 64-dim half of a block     */
constexpr int NT       = 2;             /* 16-column tiles per wave                */
constexpr float kLazy  = 8.0f;          /* headroom in log2 units (P <= 2^8)        */

struct PrefillExtParams {
    const float *q;     /* [n_seq][n_tok][n_head_q][HD] fp32                        */
    const uint16_t *k;  /* seq s at k + s*kv_seq_stride: [row][n_head_kv][HD]       */
    const uint16_t *v;
    const float *gate;  /* [n_seq][n_tok][n_head_q] or null                          */
    float *out;         /* [n_seq][n_tok][n_head_q][HD]                             */
    uint64_t kv_seq_stride;
    uint32_t n_seq, n_tok, pos_0, kv_pos0, window, n_head_q, n_head_kv, kv_mul, tq, n_qtiles;
    uint32_t chain;     /* consecutive query tiles per workgroup                    */
    uint32_t n_light;   /* tiles 0 .. n_light - 1 (window cut short by the sequence
                           start) run first; 0 keeps heaviest-first            */
    int gate_is_logit;
    float qmul;         /* softmax scale * log2(e), applied to Q before its fp16 rounding */
};

__device__ __forceinline__ half8_t as_half8(u32x4_t v) { return __builtin_bit_cast(half8_t, v); }

__device__ __forceinline__ float4_t mfma(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

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

__device__ __forceinline__ float max3(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }

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

/* Key-block geometry of query tile qt (positions t0 .. t0 + tq - 1): key
 * rows [r_lo, r_hi) of the buffer in 32-key blocks [b_lo, b_hi), of which
 * [u0, u1) need no per-key test -- every key >= the highest row's window
 * start and <= the lowest row. */
struct TileGeom {
    uint32_t t0, lo_pos, hi_pos, r_hi, b_lo, b_hi, u0, u1;
};

__device__ __forceinline__ TileGeom tile_geom(const PrefillExtParams &P, uint32_t qt) {
    TileGeom t;
    t.t0     = qt * P.tq;
    t.lo_pos = P.pos_0 + t.t0;
    t.hi_pos = P.pos_0 + min(t.t0 + P.tq, P.n_tok) - 1u;
    t.r_hi   = t.hi_pos + 1u - P.kv_pos0;
    uint32_t first_key = P.window && t.lo_pos + 1u > P.window ? t.lo_pos + 1u - P.window : 0u;
    first_key          = max(first_key, P.kv_pos0);
    t.b_lo             = (first_key - P.kv_pos0) / KB;
    t.b_hi             = (t.r_hi + KB - 1u) / KB;
    const uint32_t free_key_lo = P.window && t.hi_pos + 1u > P.window ? t.hi_pos + 1u - P.window : 0u;
    const uint32_t b_free = free_key_lo > P.kv_pos0 ? (free_key_lo - P.kv_pos0 + KB - 1u) / KB : 0u;
    const uint32_t b_diag = (t.lo_pos - P.kv_pos0 + 1u) / KB;
    t.u0 = min(max(t.b_lo, b_free), t.b_hi);
    t.u1 = max(t.u0, min(t.b_hi, b_diag));
    return t;
}

/* HD 128 (LFM3 layers) or 64: blocks of NH = HD / 64 halves for K, then V.
 * A workgroup takes a chain of P.chain consecutive query tiles of one
 * (sequence, KV head) (one tile for full layers): the blocks of its tiles
 * form one stream through the LDS ring, so the next tile's first blocks are
 * in flight while the current tile finishes, and a sliding-window tile --
 * about window / 32 blocks -- does not pay the workgroup's set-up and the
 * ring's fill on its own. */
template <int HD>
__global__ __launch_bounds__(256, HD == 64 ? 3 : 2) void k_prefill_ext(const PrefillExtParams P) {
    constexpr int NH   = HD / 64;            /* 64-dim halves per row              */
    constexpr int BLKB = 2 * NH * HALFB;     /* K halves, then V halves            */
    constexpr int NS   = HD / 32;            /* k-steps of Q.K^T                   */
    constexpr int NM   = HD / 16;            /* 16-dim tiles of O^T                */
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NBUF * BLKB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    /* 1-D grid, heaviest chains first; consecutive workgroups take
     * consecutive (sequence, KV head) pairs.  With n_light > 0 (one tile per
     * workgroup, sliding window) the short tiles at the sequence start come
     * first, longest of them first: on a CU whose first workgroup has such a
     * tile the next one starts part-way through its partner's tile, so the
     * two no longer load Q at the same time (on MI355X, B 4 x 4096, window
     * 256: 76.1 against 77.4 us; the short tiles in the second or fourth
     * round of workgroups measured 78.5 and 78.2 us). */
    const uint32_t pairs    = P.n_head_kv * P.n_seq;
    const uint32_t n_chains = (P.n_qtiles + P.chain - 1u) / P.chain;
    const uint32_t slot     = blockIdx.x / pairs;
    const uint32_t chain    = slot < P.n_light ? P.n_light - 1u - slot : n_chains - 1u - (slot - P.n_light);
    const uint32_t pair     = blockIdx.x % pairs;
    const uint32_t kvh = pair % P.n_head_kv, s = pair / P.n_head_kv;
    const uint32_t qt_first = chain * P.chain, qt_end = min(qt_first + P.chain, P.n_qtiles);

    const uint16_t *kc = P.k + (size_t)s * P.kv_seq_stride + (size_t)kvh * HD;
    const uint16_t *vc = P.v + (size_t)s * P.kv_seq_stride + (size_t)kvh * HD;
    const size_t row   = (size_t)P.n_head_kv * HD;

    /* ---- staging: the K part of a block (NH halves of 4 KB) is NH * 4
     * pieces of 1 KB; wave w fetches pieces w + 4 e (e < NH) of it and of the
     * V part.  Lane l's 16 B land at byte u = 1024 (w + 4 e) + 16 l: half
     * u / HALFB, row r = (u % HALFB) / 128, slot j = (u % 128) / 16, holding
     * the row's global chunk 8 * half + (j ^ swz(r)) */
    uint32_t st_row[NH], st_col[NH];
#pragma unroll
    for (int e = 0; e < NH; ++e) {
        const uint32_t u = 1024u * (uint32_t)(wave + 4 * e) + 16u * (uint32_t)lane;
        const uint32_t r = (u % HALFB) / 128u, j = (u % 128u) / 16u;
        st_row[e] = r;
        st_col[e] = 8u * (8u * (u / HALFB) + (j ^ (r & 7u))); /* halfs within the head's row */
    }
    const uint32_t wv       = __builtin_amdgcn_readfirstlane((uint32_t)wave);
    const uint32_t ring_lds = (uint32_t)(uintptr_t)ring; /* LDS address of the ring */

    /* ---- the block stream: block j (over the chain's tiles in order) sits
     * in ring slot j % NBUF; the fetch cursor runs two blocks ahead of the
     * block being entered */
    uint32_t n_stream = 0;
    for (uint32_t qt = qt_first; qt < qt_end; ++qt) {
        const TileGeom t = tile_geom(P, qt);
        n_stream += t.b_hi - t.b_lo;
    }
    uint32_t f_qt = qt_first, f_j = 0;
    TileGeom fg   = tile_geom(P, f_qt);
    uint32_t f_b  = fg.b_lo;
    /* 2 NH fetches per wave and block (vmcnt counts them) */
    auto fetch_next = [&]() {
        const uint32_t slot = ring_lds + (f_j % NBUF) * BLKB;
        const uint32_t b    = f_b;
        if ((b + 1u) * KB <= fg.r_hi) {
            /* a whole block: uniform base, fixed per-lane offsets */
            const size_t boff = (size_t)b * KB * row;
#pragma unroll
            for (int e = 0; e < NH; ++e) {
                const uint32_t voff  = (st_row[e] * (uint32_t)row + st_col[e]) * (uint32_t)sizeof(uint16_t);
                const uint32_t piece = slot + 1024u * (wv + 4u * (uint32_t)e);
                fetch16_lds(voff, kc + boff, piece);
                fetch16_lds(voff, vc + boff, piece + (uint32_t)(NH * HALFB));
            }
        } else {
#pragma unroll
            for (int e = 0; e < NH; ++e) {
                uint32_t r = b * KB + st_row[e];
                r = r < fg.r_hi ? r : fg.r_hi - 1u; /* rows past the keys: masked */
                const size_t off     = (size_t)r * row + st_col[e];
                const uint32_t piece = slot + 1024u * (wv + 4u * (uint32_t)e);
                fetch16_lds(kc + off, piece);
                fetch16_lds(vc + off, piece + (uint32_t)(NH * HALFB));
            }
        }
        ++f_j;
        if (++f_b == fg.b_hi && ++f_qt < qt_end) {
            fg  = tile_geom(P, f_qt);
            f_b = fg.b_lo;
        }
    };

    /* the first two blocks are in flight before the first tile's Q loads:
     * the wait for Q (which also covers these older fetches) then takes one
     * memory round trip, not two */
    fetch_next();
    if (n_stream > 1u) fetch_next();

    /* fragment offsets within a 64-dim half (bytes).  K: row 16*mt + l16,
     * chunk 4*(st % 2) + g.  V (transposing read): lane l16 of group g
     * addresses row 4g + l16/4 of a 16-key half, dims 16*mt + 4*(l16 % 4) */
    const uint32_t kswz  = (uint32_t)(g ^ (l16 & 7));
    const uint32_t koff0 = (uint32_t)l16 * 128u + 16u * kswz;
    const uint32_t koff1 = (uint32_t)l16 * 128u + 16u * (kswz ^ 4u);
    const uint32_t vr    = (uint32_t)(4 * g + (l16 >> 2)); /* V row read (its + 16 twin has the same swizzle) */
    uint32_t voff[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
        voff[mt] = vr * 128u + 16u * ((2u * (uint32_t)mt + (uint32_t)((l16 >> 1) & 1)) ^ (vr & 7u)) + 8u * (l16 & 1);
    const half8_t ones8 = (half8_t)(_Float16)1.0f;

    /* Q (fp32) and the output gates of a tile: all loads are issued before
     * any is used (qp is a valid row for a padding column too; its values
     * are zeroed after): with a use between them the compiler waited for
     * each column tile's loads, one memory round trip per tile.  In a chain
     * the next tile's loads are issued before the current tile's last P.V
     * (its Q fragments and one score set are dead by then), so they land
     * while that step and the epilogue run. */
    float4 qraw[NT][NS][2];
    float gnext[NT];
    auto load_q = [&](uint32_t qt_) {
        const uint32_t t0_ = qt_ * P.tq;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const uint32_t c = (uint32_t)(wave * 32 + nt * 16 + l16);
            const uint32_t j = c / P.tq, t = t0_ + c % P.tq;
            const bool ok    = t < P.n_tok;
            gnext[nt] = (P.gate && ok) ? P.gate[((size_t)s * P.n_tok + t) * P.n_head_q + kvh * P.kv_mul + j] : 1.0f;
            const float *qp =
                P.q + (((size_t)s * P.n_tok + (ok ? t : 0u)) * P.n_head_q + kvh * P.kv_mul + j) * HD + 8 * g;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                qraw[nt][st][0] = *reinterpret_cast<const float4 *>(qp + 32 * st);
                qraw[nt][st][1] = *reinterpret_cast<const float4 *>(qp + 32 * st + 4);
            }
        }
    };
    load_q(qt_first);

    uint32_t j0 = 0; /* stream index of the current tile's first block */
    for (uint32_t qt = qt_first; qt < qt_end; ++qt) {
        const TileGeom tg = tile_geom(P, qt);
        const uint32_t t0 = tg.t0;
        auto block_masked = [&](uint32_t b) { return b < tg.u0 || b >= tg.u1; };
        auto block_lds    = [&](uint32_t b) { return ring + ((j0 + b - tg.b_lo) % NBUF) * BLKB; };

        /* ---- columns of this lane: (head j, row t) per N-tile -------------- */
        uint32_t col_pos[NT], col_lo[NT];
        bool col_ok[NT];
        half8_t qf[NT][NS];
        float graw[NT]; /* the output gates (loaded with Q): the epilogue does not wait for them */
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const uint32_t c = (uint32_t)(wave * 32 + nt * 16 + l16);
            const uint32_t t = t0 + c % P.tq;
            col_ok[nt]  = t < P.n_tok;
            graw[nt]    = gnext[nt];
            col_pos[nt] = P.pos_0 + t;
            col_lo[nt]  = (P.window && col_pos[nt] + 1u > P.window) ? col_pos[nt] + 1u - P.window : 0u;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const float4 a = qraw[nt][st][0], b = qraw[nt][st][1];
                const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                half8_t h;
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = col_ok[nt] ? (_Float16)(x[e] * P.qmul) : (_Float16)0.0f;
                qf[nt][st] = h;
            }

        float4_t oacc[NM][NT];
        float4_t negm[NT];
        float4_t lacc[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            negm[nt] = (float4_t)0.0f;
            lacc[nt] = (float4_t)0.0f;
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] = (float4_t)0.0f;
        }

        /* S^T of block b: two 16-key tiles x NT column tiles */
        auto scores = [&](auto mask_tag, uint32_t b, float4_t (&sc)[2][NT]) {
            constexpr bool MASK = decltype(mask_tag)::value;
            const uint8_t *kb = block_lds(b);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                half8_t kf[NS];
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    kf[2 * h]     = as_half8(*reinterpret_cast<const u32x4_t *>(kb + h * HALFB + mt * 16 * 128 + koff0));
                    kf[2 * h + 1] = as_half8(*reinterpret_cast<const u32x4_t *>(kb + h * HALFB + mt * 16 * 128 + koff1));
                }
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    float4_t a = mfma(kf[0], qf[nt][0], negm[nt]);
#pragma unroll
                    for (int st = 1; st < NS; ++st) a = mfma(kf[st], qf[nt][st], a);
                    sc[mt][nt] = a;
                }
            }
            if constexpr (MASK) {
                /* element (mt, i) is key key0 + 16 mt + i of the column */
                const int key0 = (int)(P.kv_pos0 + b * KB) + 4 * g;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const int hi = (int)col_pos[nt] - key0, lo = (int)col_lo[nt] - key0;
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (16 * mt + i > hi || 16 * mt + i < lo) sc[mt][nt][i] = -INFINITY;
                }
            }
        };

        /* lazy max per column: m is set by the first block holding one of the
         * column's keys (its exact maximum there) and raised later only when a
         * block exceeds it by more than kLazy, rescaling O, l and the pending
         * scores (a rare, wave-uniform branch).  With a window, a column's first
         * keys may lie in a later block than the tile's first; until then its
         * scores are all masked, p = 0 and O = l = 0, so setting m needs no
         * rescale (and exp2(-m) could overflow). */
        bool mset[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) mset[nt] = false;
        auto update_max = [&](float4_t (&sc)[2][NT]) {
            float mx[NT];
            bool any_raise = false;
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                float v = max3(max3(sc[0][nt][0], sc[0][nt][1], sc[0][nt][2]), sc[0][nt][3], sc[1][nt][0]);
                v = max3(max3(v, sc[1][nt][1], sc[1][nt][2]), sc[1][nt][3], -INFINITY);
                mx[nt] = v;
                any_raise |= v > kLazy || (!mset[nt] && v > -INFINITY);
            }
            if (__builtin_amdgcn_ballot_w64(any_raise) != 0ull) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    float v = mx[nt]; /* column max over the 4 lanes holding it */
                    v = fmaxf(v, __shfl_xor(v, 16));
                    v = fmaxf(v, __shfl_xor(v, 32));
                    const bool raise  = v > kLazy || (!mset[nt] && v > -INFINITY);
                    const float inc   = raise ? v : 0.0f;
                    const float alpha = mset[nt] ? __builtin_amdgcn_exp2f(-inc) : 1.0f;
                    mset[nt] = mset[nt] || raise;
                    negm[nt] -= inc;
                    lacc[nt] *= alpha;
                    sc[0][nt] -= inc;
                    sc[1][nt] -= inc;
#pragma unroll
                    for (int mt = 0; mt < NM; ++mt) oacc[mt][nt] *= alpha;
                }
            }
        };

        auto accumulate = [&](uint32_t b, const float4_t (&sc)[2][NT]) {
            u32x4_t pf[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const float4_t a = sc[0][nt], c = sc[1][nt];
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
            const uint8_t *vb = block_lds(b) + NH * HALFB;
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const uint8_t *vh = vb + (mt >> 2) * HALFB;
                const half4_t lo  = lds_read_tr(vh + voff[mt & 3]);
                const half4_t hi  = lds_read_tr(vh + 16 * 128 + voff[mt & 3]);
                const half8_t av  = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) oacc[mt][nt] = mfma(av, as_half8(pf[nt]), oacc[mt][nt]);
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) lacc[nt] = mfma(ones8, as_half8(pf[nt]), lacc[nt]);
        };

        /* entering block b (at the start of step b - 1, before S^T(b)): this
         * wave's fetches of block b have landed (those of the next stream
         * block may still be in flight), and the barrier makes every wave's
         * part visible.  The previous stream block is still in use (P.V of the
         * previous step); the ring slot two blocks ahead held the block two
         * behind, which every wave finished before the barrier, so the stream
         * block two ahead -- of this tile or the next -- is fetched into it. */
        auto enter_block = [&](uint32_t b) {
            const uint32_t j = j0 + b - tg.b_lo;
            if (j + 1u < n_stream) {
                if constexpr (NH == 2) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            __syncthreads();
            if (j + 2u < n_stream) fetch_next();
        };

        const uint32_t b_lo = tg.b_lo, b_hi = tg.b_hi, u0 = tg.u0, u1 = tg.u1;
        enter_block(b_lo);
        float4_t scur[2][NT];
        if (block_masked(b_lo)) scores(std::true_type{}, b_lo, scur);
        else scores(std::false_type{}, b_lo, scur);
        update_max(scur);
        /* step b: S^T(b + 1) into the other register set, then P(b) and PV(b);
         * two steps per iteration with the sets swapping roles */
        float4_t snxt[2][NT];
        auto step = [&](auto mask_tag, uint32_t b, float4_t(&sc)[2][NT], float4_t(&sn)[2][NT])
                        __attribute__((always_inline)) {
            enter_block(b + 1u);
            scores(mask_tag, b + 1u, sn);
            accumulate(b, sc);
            update_max(sn);
        };
        uint32_t b = b_lo;
        /* steps b .. b_end - 1; S^T(b) is in scur on entry and on exit */
        auto run_steps = [&](auto mask_tag, uint32_t b_end) __attribute__((always_inline)) {
            for (; b + 2u <= b_end; b += 2u) {
                step(mask_tag, b, scur, snxt);
                step(mask_tag, b + 1u, snxt, scur);
            }
            if (b < b_end) {
                step(mask_tag, b, scur, snxt);
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) scur[mt][nt] = snxt[mt][nt];
                ++b;
            }
        };
        /* blocks [u0, u1) need no mask; masked ones sit below (window edge)
         * and above (diagonal) */
        run_steps(std::true_type{}, u0 > 0u ? u0 - 1u : 0u);
        run_steps(std::false_type{}, u1 > 0u ? u1 - 1u : 0u);
        run_steps(std::true_type{}, b_hi - 1u);
        /* the next tile's Q loads before the last P.V; on the chain's last
         * tile the Q registers are cleared instead, so that no path carries
         * the loaded values through a whole tile (a conditional load alone
         * kept them live, and the kernel spilled) */
        if (qt + 1u < qt_end) {
            load_q(qt + 1u);
        } else {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                gnext[nt] = 0.0f;
#pragma unroll
                for (int st = 0; st < NS; ++st) qraw[nt][st][0] = qraw[nt][st][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        accumulate(b, scur);
        /* ---- epilogue: O * gate / l ------------------------------------------ */
        float inv[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const float lt = lacc[nt][0];
            float gv       = 1.0f;
            if (P.gate) {
                const float gl = graw[nt];
                gv             = P.gate_is_logit ? 1.0f / (1.0f + expf(-gl)) : gl;
            }
            inv[nt] = lt > 0.0f ? gv / lt : 0.0f;
        }
        if (HD == 128 && qt + 1u >= qt_end) {
            /* (head_dim 128: the head_dim-64 instance, at three waves per SIMD,
             * has no registers to spare for it.)
             * The workgroup's last tile: the ring is free once every wave's
             * last P.V has read it (no fetch is outstanding), so each wave
             * stages its 32 output rows there row-major and stores whole
             * rows: one store instruction covers 64 / CHK rows of HD fp32,
             * where the fragment layout covers 16 rows x 64 B per
             * instruction (half of each 128-B line).  Row r's 16-B chunk q
             * sits at slot q ^ (r & 15): conflict-free for both the fragment
             * writes and the row reads. */
            constexpr int CHK = HD / 4; /* 16-B chunks per output row */
            __syncthreads();
            uint8_t *ob = ring + (size_t)wave * 32u * (uint32_t)(HD * 4);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const uint32_t r = (uint32_t)(nt * 16 + l16);
#pragma unroll
                for (int mt = 0; mt < NM; ++mt) {
                    const uint32_t q = (uint32_t)(4 * mt + g);
                    *reinterpret_cast<float4_t *>(ob + r * (uint32_t)(HD * 4) + 16u * (q ^ (r & 15u))) =
                        oacc[mt][nt] * inv[nt];
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); /* this wave's rows are in LDS */
            constexpr int RPI = 64 / CHK;                       /* rows per store instruction */
            const uint32_t lg = (uint32_t)__builtin_ctz(P.tq); /* tq = 128 / kv_mul: a power of two */
#pragma unroll 2
            for (int k = 0; k < 32 / RPI; ++k) {
                const uint32_t r = (uint32_t)(k * RPI + lane / CHK), q = (uint32_t)(lane % CHK);
                const uint32_t c = (uint32_t)(wave * 32) + r;
                const uint32_t j = c >> lg, t = t0 + (c & (P.tq - 1u));
                const float4_t v = *reinterpret_cast<const float4_t *>(ob + r * (uint32_t)(HD * 4) + 16u * (q ^ (r & 15u)));
                if (t < P.n_tok)
                    *reinterpret_cast<float4_t *>(P.out + (((size_t)s * P.n_tok + t) * P.n_head_q + kvh * P.kv_mul + j) * HD +
                                                  4u * q) = v;
            }
            break;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            if (!col_ok[nt]) continue;
            const uint32_t c  = (uint32_t)(wave * 32 + nt * 16 + l16);
            const uint32_t j  = c / P.tq, t = t0 + c % P.tq;
            float *op = P.out + (((size_t)s * P.n_tok + t) * P.n_head_q + kvh * P.kv_mul + j) * HD;
#pragma unroll
            for (int mt = 0; mt < NM; ++mt)
                *reinterpret_cast<float4 *>(op + 16 * mt + 4 * g) =
                    make_float4(oacc[mt][nt][0] * inv[nt], oacc[mt][nt][1] * inv[nt], oacc[mt][nt][2] * inv[nt],
                                oacc[mt][nt][3] * inv[nt]);
        }
        j0 += b_hi - b_lo;
    }
}

} // namespace

/* Query tiles per workgroup: one unless set by lfm_attn_set_tuning.  On
 * MI355X the sliding-window workload (B 4 x 4096, 16q/4kv, window 256) took
 * 82.2 us with one tile per workgroup, 87.0 us with chains of 2, 89.1 us
 * with chains of 4 and 102 us with chains of 8, with the next tile's Q in
 * flight during each tile's last step (before that prefetch: 84.5 and
 * 89.6 us for 2 and 4): the single-tile workgroups already hide each
 * other's set-up, and a static chain per workgroup loses the dynamic
 * balance of 2048 short workgroups over the CUs.  Full layers (window 0 or
 * above 32 tiles) always take one tile per workgroup. */
static uint32_t prefill_chain(uint32_t window, uint32_t tq, uint32_t n_qtiles) {
    if (!window || window > 32u * tq) return 1u;
    const uint32_t forced = current_tuning().prefill_chain; /* tests, tuning */
    return forced ? min(forced, n_qtiles) : 1u;
}

PrefillExtPlan prefill_ext_plan(uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint32_t window, uint32_t n_head_q,
                                uint32_t n_head_kv) {
    PrefillExtPlan pl{};
    pl.tq       = 128u / (n_head_q / n_head_kv);
    const uint32_t n_qtiles = (n_tok + pl.tq - 1u) / pl.tq;
    pl.chain    = prefill_chain(window, pl.tq, n_qtiles);
    /* tiles whose window reaches before the sequence start (first row's
     * position + 1 < window): the first ceil((window - pos_0 - 1) / tq) */
    pl.n_light  = (pl.chain == 1u && window > pos_0 + 1u) ? min(n_qtiles, (window - pos_0 - 1u + pl.tq - 1u) / pl.tq)
                                                          : 0u;
    pl.n_wg     = ((n_qtiles + pl.chain - 1u) / pl.chain) * n_head_kv * n_seq;
    return pl;
}

bool prefill_ext_supports(uint32_t head_dim, uint32_t kv_mul) {
    return (head_dim == 128u || head_dim == 64u) && kv_mul >= 1u && kv_mul <= 32u && (128u % kv_mul) == 0u;
}

int launch_prefill_ext(const float *q, const uint16_t *k, const uint16_t *v, const float *gate, int gate_is_logit,
                       float *out, uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint32_t kv_pos0,
                       uint64_t kv_seq_stride, uint32_t window, uint32_t n_head_q, uint32_t n_head_kv,
                       uint32_t head_dim, float scale, hipStream_t stream) {
    PrefillExtParams P{};
    P.q             = q;
    P.k             = k;
    P.v             = v;
    P.gate          = gate;
    P.gate_is_logit = gate_is_logit;
    P.out           = out;
    P.kv_seq_stride = kv_seq_stride;
    P.n_seq         = n_seq;
    P.n_tok         = n_tok;
    P.pos_0         = pos_0;
    P.kv_pos0       = kv_pos0;
    P.window        = window;
    P.n_head_q      = n_head_q;
    P.n_head_kv     = n_head_kv;
    P.kv_mul        = n_head_q / n_head_kv;
    const PrefillExtPlan pl = prefill_ext_plan(n_seq, n_tok, pos_0, window, n_head_q, n_head_kv);
    P.tq            = pl.tq;
    P.n_qtiles      = (n_tok + P.tq - 1u) / P.tq;
    P.qmul          = scale * kLog2e;
    P.chain         = pl.chain;
    P.n_light       = pl.n_light;
    const uint32_t n_wg = pl.n_wg;
    hipEvent_t ev0, ev1;
    profile_events(&ev0, &ev1);
    if (ev0) (void)hipEventRecord(ev0, stream);
    if (head_dim == 128u)
        hipLaunchKernelGGL(k_prefill_ext<128>, dim3(n_wg), dim3(256), 0, stream, P);
    else
        hipLaunchKernelGGL(k_prefill_ext<64>, dim3(n_wg), dim3(256), 0, stream, P);
    hipError_t e = hipGetLastError();
    if (ev1) (void)hipEventRecord(ev1, stream);
    return hip_status(e);
}

} // namespace lfm
