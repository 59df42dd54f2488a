/*
 * fnv_hash.hip -- FNV-1a 64 of a device buffer, computed in parallel.
 *
 * The .lfmcache trailer is FNV-1a 64 over the payload
 * (lfm2_fnv1a_update, tools/lfm2_sys_cache.c:382-389):
 *     h <- (h XOR byte) * P  (mod 2^64),  P = 2^40 + 435.
 * One byte per step and a dependent multiply: about 0.7 GB/s on one core.
 *
 * Two facts make it parallel:
 *  (1) The low byte s = h mod 256 evolves on its own:
 *          s' = ((s XOR b) * 179) mod 256          (435 mod 256 = 179)
 *      so each run of bytes acts on s as a permutation of 256 states, and
 *      runs compose.
 *  (2) XOR with a byte moves h by d = (s XOR b) - s, a small signed number,
 *      so h_n = h_0 P^n + sum_j d_j P^(n-j): a polynomial in P once the
 *      states s_j are known.
 *
 * Kernels:
 *  k_fnv_maps     one wave per 1 KiB chunk: the chunk's 256-state map.
 *                 Flipping bit 7 of s flips bit 7 of s' and nothing else
 *                 (128 * 179 = 128 mod 256), so map(s ^ 128) = map(s) ^ 128
 *                 and only states 0..127 are run: two per lane in 16-bit
 *                 halves (v_pk_mul_lo_u16; the low byte of a 16-bit product
 *                 depends only on low bytes, so masking waits until the end).
 *  k_fnv_compose  groups of 64 maps: per group-start state, the state at the
 *                 start of every member (written over the member maps) and
 *                 the group's map (input to the next level).
 *  k_fnv_poly     one lane per chunk: the chunk's start state from the
 *                 prefix tables (one lookup per level), then a Horner pass
 *                 over its bytes for sum d_j P^(len-j), weighted by
 *                 P^(bytes after the chunk) and summed (mod 2^64).
 * Workspace: 256 B per chunk (a quarter of the data) plus the upper levels.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace lfm {
namespace {

constexpr uint32_t kChunk   = 1024u;
constexpr uint32_t kFanIn   = 64u;
constexpr uint32_t kMaxLvls = 8u;
constexpr uint64_t kPrime   = 0x100000001B3ull;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint64_t mul_p(uint64_t x) { return x * 435ull + (x << 40); }

__device__ uint64_t pow_p(uint64_t e) {
    uint64_t r = 1ull, b = kPrime;
    while (e) {
        if (e & 1ull) r *= b;
        b *= b;
        e >>= 1;
    }
    return r;
}

/* 256-state map of each 1 KiB chunk: maps[c][s] = low byte after the chunk
 * starting from low byte s.  64 lanes run states (2t, 2t+1); states
 * 128 + (2t, 2t+1) follow by the bit-7 symmetry. */
__global__ __launch_bounds__(64) void k_fnv_maps(const uint8_t *__restrict__ data, uint64_t len,
                                                  uint8_t *__restrict__ maps, uint64_t *__restrict__ acc_out) {
    const uint64_t c0 = (uint64_t)blockIdx.x * kChunk;
    const uint32_t n  = (uint32_t)(len - c0 < kChunk ? len - c0 : kChunk);
    const uint32_t t  = threadIdx.x;
    if (blockIdx.x == 0u && t == 0u) *acc_out = 0ull;
    u16x2 s = {(unsigned short)(2u * t), (unsigned short)(2u * t + 1u)};
    const u16x2 m = {179, 179};
    const uint32_t *w = (const uint32_t *)(data + c0);
    const uint32_t nw = n / 4u;
#pragma unroll 4
    for (uint32_t i = 0; i < nw; ++i) {
        const uint32_t v = w[i];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const unsigned short b = (unsigned short)((v >> (8 * k)) & 0xffu);
            s                      = (s ^ (u16x2){b, b}) * m;
        }
    }
    for (uint32_t i = nw * 4u; i < n; ++i) {
        const unsigned short b = data[c0 + i];
        s                      = (s ^ (u16x2){b, b}) * m;
    }
    const uint32_t out = (uint32_t)(s.x & 0xffu) | ((uint32_t)(s.y & 0xffu) << 8);
    uint16_t *row      = (uint16_t *)(maps + (size_t)blockIdx.x * 256u);
    row[t]             = (uint16_t)out;
    row[64u + t]       = (uint16_t)(out ^ 0x8080u);
}

/* Group of up to 64 maps: member maps become prefix tables (state at the
 * member's start for each group-start state); the group map goes to up. */
__global__ __launch_bounds__(256) void k_fnv_compose(uint8_t *__restrict__ maps, uint32_t n,
                                                     uint8_t *__restrict__ up) {
    __shared__ uint8_t lds[kFanIn * 256u];
    const uint32_t g0  = blockIdx.x * kFanIn;
    const uint32_t cnt = n - g0 < kFanIn ? n - g0 : kFanIn;
    const uint32_t t   = threadIdx.x;
    const uint4 *src   = (const uint4 *)(maps + (size_t)g0 * 256u);
    for (uint32_t i = t; i < cnt * 16u; i += 256u) ((uint4 *)lds)[i] = src[i];
    __syncthreads();
    uint32_t cur = t;
    for (uint32_t j = 0; j < cnt; ++j) {
        maps[(size_t)(g0 + j) * 256u + t] = (uint8_t)cur;
        cur = lds[j * 256u + cur];
    }
    up[(size_t)blockIdx.x * 256u + t] = (uint8_t)cur;
}

struct PolyParams {
    const uint8_t *data;
    uint64_t len;
    uint32_t n_chunks;
    uint32_t n_levels;               /* prefix levels (0: a single chunk) */
    const uint8_t *prefix[kMaxLvls]; /* level l: one 256-entry table per element */
    uint32_t start_state;
    uint64_t *acc;
};

__global__ __launch_bounds__(256) void k_fnv_poly(PolyParams p) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t part    = 0ull;
    if (i < p.n_chunks) {
        uint32_t s = p.start_state;
        for (int l = (int)p.n_levels - 1; l >= 0; --l) {
            const uint32_t j = i >> (6u * (uint32_t)l);
            s                = p.prefix[l][(size_t)j * 256u + s];
        }
        const uint64_t c0  = (uint64_t)i * kChunk;
        const uint32_t n   = (uint32_t)(p.len - c0 < kChunk ? p.len - c0 : kChunk);
        const uint4 *src   = (const uint4 *)(p.data + c0);
        uint64_t a         = 0ull;
        const uint32_t n16 = n / 16u;
        for (uint32_t q = 0; q < n16; ++q) {
            const uint4 v          = src[q];
            const uint32_t wd[4]   = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const uint32_t b = (wd[k >> 2] >> (8 * (k & 3))) & 0xffu;
                const uint32_t x = s ^ b;
                a                = mul_p(a + (uint64_t)(int64_t)((int32_t)x - (int32_t)s));
                s                = (x * 179u) & 0xffu;
            }
        }
        for (uint32_t q = n16 * 16u; q < n; ++q) {
            const uint32_t x = s ^ p.data[c0 + q];
            a                = mul_p(a + (uint64_t)(int64_t)((int32_t)x - (int32_t)s));
            s                = (x * 179u) & 0xffu;
        }
        part = a * pow_p(p.len - c0 - n);
    }
    /* wave sum mod 2^64, one atomic per wave */
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)part, off, 64);
        const uint32_t hi = __shfl_xor((uint32_t)(part >> 32), off, 64);
        part += ((uint64_t)hi << 32) | lo;
    }
    if ((threadIdx.x & 63u) == 0u && part) atomicAdd((unsigned long long *)p.acc, (unsigned long long)part);
}

} // namespace

size_t fnv1a64_workspace_bytes(uint64_t len) {
    uint64_t n = (len + kChunk - 1u) / kChunk, total = 256u; /* acc slot */
    while (n > 1u) {
        total += n * 256u;
        n = (n + kFanIn - 1u) / kFanIn;
    }
    return (size_t)(total + 256u);
}

/* Enqueues the hash of len > 0 bytes (16-byte aligned) continuing from h_in;
 * the polynomial part lands in the first 8 bytes of ws (fnv1a64_finish). */
int launch_fnv1a64(const void *data, uint64_t len, uint64_t h_in, void *ws, hipStream_t stream) {
    uint64_t *acc_dev = (uint64_t *)ws;
    if (len == 0u) return -1;
    uint32_t n = (uint32_t)((len + kChunk - 1u) / kChunk);
    uint8_t *w = (uint8_t *)ws + 256u;
    PolyParams p{};
    p.data        = (const uint8_t *)data;
    p.len         = len;
    p.n_chunks    = n;
    p.start_state = (uint32_t)(h_in & 0xffu);
    p.acc         = acc_dev;
    hipLaunchKernelGGL(k_fnv_maps, dim3(n), dim3(64), 0, stream, (const uint8_t *)data, len, w, acc_dev);
    uint32_t lv = 0;
    while (n > 1u) {
        if (lv == kMaxLvls) return -1;
        const uint32_t up_n = (n + kFanIn - 1u) / kFanIn;
        uint8_t *up         = w + (size_t)n * 256u;
        hipLaunchKernelGGL(k_fnv_compose, dim3(up_n), dim3(256), 0, stream, w, n, up);
        p.prefix[lv++] = w;
        w              = up;
        n              = up_n;
    }
    p.n_levels = lv;
    hipLaunchKernelGGL(k_fnv_poly, dim3((p.n_chunks + 255u) / 256u), dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

/* h_in * P^len + acc (mod 2^64): the hash after len bytes from h_in. */
uint64_t fnv1a64_finish(uint64_t h_in, uint64_t len, uint64_t acc) {
    uint64_t r = 1ull, b = kPrime, e = len;
    while (e) {
        if (e & 1ull) r *= b;
        b *= b;
        e >>= 1;
    }
    return h_in * r + acc;
}

} // namespace lfm
