/*
 * kv_shift.hip -- attention-sink eviction on the device-resident fp16 KV
 * caches: rows move down by n_discard positions and every moved key is
 * counter-rotated by -n_discard positions.
 *
 * Semantics: lfm2_kv_cache_shift_sinks_avx2
 * (tools/lfm2_runtime_features.c:744-833) and lfm3_kv_cache_shift_sinks
 * (tools/lfm2_runtime_features.c:1055-1163).  For a key pair (lo, hi) =
 * (k[i], k[i + d/2]) and the table row of position n_discard (c, s):
 *     lo' = fma(lo, c, hi*s)      hi' = fma(hi, c, -(lo*s))
 * in fp32, stored fp16 round-to-nearest-even -- the AVX2 kernels' operation
 * order (_mm256_fmadd_ps(lo, c, _mm256_mul_ps(hi, s)) and the matching
 * fmsub), so results are bit-identical.  Values move unchanged.
 *
 * One kernel moves rows under three row maps:
 *   SHIFT   dst = dst0 + i, src = dst + src_delta, keys rotated.  A shift
 *           whose source and destination ranges overlap is issued in chunks
 *           of at most src_delta rows, in order on one stream, so no chunk
 *           reads a row an earlier chunk wrote.
 *   GATHER  (SWA ring) dst = staging row i; position t = t_start + i moves
 *           from ring slot (t >= n_sink ? t + n_discard : t) % cap, rotated
 *           when t >= n_sink.
 *   SCATTER staging row i -> ring slot (t_start + i) % cap.
 * Each thread moves 8 rotation pairs of one head: 2 x 16 B of K and the two
 * matching 16-B chunks of V.  HBM-bound: 4 bytes moved per cache byte.
 */
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "lfm_attn.h"

namespace lfm {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

enum : uint32_t { MAP_SHIFT = 0, MAP_GATHER = 1, MAP_SCATTER = 2 };

struct MoveParams {
    const uint16_t *k_src, *v_src;
    uint16_t *k_dst, *v_dst;
    const float *cos, *sin; /* table row of position n_discard, head_dim/2 entries */
    uint32_t kv_dim, head_dim, n_rows, map;
    uint32_t dst0, src_delta;            /* SHIFT */
    uint32_t t_start, n_sink, n_discard, cap; /* GATHER / SCATTER */
};

__global__ __launch_bounds__(256) void k_kv_move(const MoveParams P) {
    const uint32_t half = P.head_dim >> 1;
    const uint32_t per_row = P.kv_dim >> 4; /* threads per row: 8 pairs each */
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t i = gid / per_row;
    if (i >= P.n_rows) return;
    const uint32_t r = gid - i * per_row;
    const uint32_t chunks = half >> 3; /* 8-pair chunks per head */
    const uint32_t h = r / chunks, c8 = r - h * chunks;

    uint32_t src, dst;
    bool rotate;
    if (P.map == MAP_SHIFT) {
        dst    = P.dst0 + i;
        src    = dst + P.src_delta;
        rotate = true;
    } else if (P.map == MAP_GATHER) {
        const uint32_t t = P.t_start + i;
        rotate = t >= P.n_sink;
        src    = (rotate ? t + P.n_discard : t) % P.cap;
        dst    = i;
    } else {
        src    = i;
        dst    = (P.t_start + i) % P.cap;
        rotate = false;
    }
    const size_t lo_off = (size_t)h * P.head_dim + 8u * c8;
    const size_t so = (size_t)src * P.kv_dim + lo_off, d_o = (size_t)dst * P.kv_dim + lo_off;

    const u32x4_t vlo = *reinterpret_cast<const u32x4_t *>(P.v_src + so);
    const u32x4_t vhi = *reinterpret_cast<const u32x4_t *>(P.v_src + so + half);
    u32x4_t klo = *reinterpret_cast<const u32x4_t *>(P.k_src + so);
    u32x4_t khi = *reinterpret_cast<const u32x4_t *>(P.k_src + so + half);
    if (rotate) {
        const half8_t lo8 = __builtin_bit_cast(half8_t, klo), hi8 = __builtin_bit_cast(half8_t, khi);
        half8_t nlo, nhi;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float c = P.cos[8u * c8 + e], s = P.sin[8u * c8 + e];
            const float lo = (float)lo8[e], hi = (float)hi8[e];
            const float hs = hi * s, ls = lo * s;
            float nl = __builtin_fmaf(lo, c, hs), nh = __builtin_fmaf(hi, c, -ls);
            /* round to fp32 first, then to fp16, like the reference's
             * fmadd + cvtps_ph: without this barrier the compiler fuses the
             * fma and the conversion into v_fma_mix{lo,hi}_f16, a single
             * rounding that differs in the last bit on ties */
            asm volatile("" : "+v"(nl), "+v"(nh));
            nlo[e] = (_Float16)nl;
            nhi[e] = (_Float16)nh;
        }
        klo = __builtin_bit_cast(u32x4_t, nlo);
        khi = __builtin_bit_cast(u32x4_t, nhi);
    }
    *reinterpret_cast<u32x4_t *>(P.k_dst + d_o)        = klo;
    *reinterpret_cast<u32x4_t *>(P.k_dst + d_o + half) = khi;
    *reinterpret_cast<u32x4_t *>(P.v_dst + d_o)        = vlo;
    *reinterpret_cast<u32x4_t *>(P.v_dst + d_o + half) = vhi;
}

int launch_move(const MoveParams &P, hipStream_t stream) {
    if (P.n_rows == 0u) return LFM_ATTN_OK;
    const uint64_t threads = (uint64_t)P.n_rows * (P.kv_dim >> 4);
    const uint32_t blocks  = (uint32_t)((threads + 255u) / 256u);
    hipLaunchKernelGGL(k_kv_move, dim3(blocks), dim3(256), 0, stream, P);
    return hip_status(hipGetLastError());
}

} // namespace

int launch_kv_shift(uint16_t *k, uint16_t *v, uint32_t kv_dim, uint32_t head_dim, uint32_t n_sink,
                    uint32_t n_keep, uint32_t n_discard, const float *cos_row, const float *sin_row,
                    hipStream_t stream) {
    MoveParams P{};
    P.k_src = k;
    P.v_src = v;
    P.k_dst = k;
    P.v_dst = v;
    P.cos = cos_row;
    P.sin = sin_row;
    P.kv_dim = kv_dim;
    P.head_dim = head_dim;
    P.map = MAP_SHIFT;
    P.src_delta = n_discard;
    /* chunks of at most n_discard rows: a chunk's sources lie above every
     * destination written so far and below none of its own */
    for (uint32_t done = 0; done < n_keep;) {
        const uint32_t n = n_keep - done < n_discard ? n_keep - done : n_discard;
        P.dst0 = n_sink + done;
        P.n_rows = n;
        const int st = launch_move(P, stream);
        if (st != LFM_ATTN_OK) return st;
        done += n;
    }
    return LFM_ATTN_OK;
}

int launch_kv_swa_repack(uint16_t *k, uint16_t *v, uint32_t kv_dim, uint32_t head_dim, uint32_t cap,
                         uint32_t t_start, uint32_t n_valid, uint32_t n_sink, uint32_t n_discard,
                         const float *cos_row, const float *sin_row, uint16_t *stage_k,
                         uint16_t *stage_v, hipStream_t stream) {
    MoveParams P{};
    P.cos = cos_row;
    P.sin = sin_row;
    P.kv_dim = kv_dim;
    P.head_dim = head_dim;
    P.n_rows = n_valid;
    P.t_start = t_start;
    P.n_sink = n_sink;
    P.n_discard = n_discard;
    P.cap = cap;
    P.k_src = k;
    P.v_src = v;
    P.k_dst = stage_k;
    P.v_dst = stage_v;
    P.map = MAP_GATHER;
    int st = launch_move(P, stream);
    if (st != LFM_ATTN_OK) return st;
    P.k_src = stage_k;
    P.v_src = stage_v;
    P.k_dst = k;
    P.v_dst = v;
    P.map = MAP_SCATTER;
    return launch_move(P, stream);
}

} // namespace lfm
