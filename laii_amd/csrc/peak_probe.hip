/*
 * peak_probe.hip -- the box's achievable denominators, measured beside the
 * attention kernels: a streaming HBM read and a dense fp16 MFMA loop.
 * They carry no reference semantics; bench.py reports them next to the
 * datasheet peaks (8 TB/s, 2.5 PFLOP/s) so each roofline fraction can also be
 * read against what this device delivers.
 *
 * k_probe_read  grid-stride 16-B loads over n16 chunks, XOR-folded so the
 *               loads stay live; one 4-byte store per workgroup.
 * k_probe_mfma  each wave runs iters rounds of 8 independent
 *               v_mfma_f32_16x16x32_f16 chains (16,384 FLOPs each) on
 *               register operands, then stores one value per lane.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace lfm {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_probe_read(const u32x4_t *__restrict__ src, uint64_t n16,
                                                    uint32_t *__restrict__ sink) {
    uint32_t acc = 0;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const u32x4_t v = __builtin_nontemporal_load(src + i);
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    __shared__ uint32_t part[4];
    if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0u) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

__global__ __launch_bounds__(256) void k_probe_mfma(float *__restrict__ out, uint32_t iters, float seed) {
    const float s = seed + (float)(threadIdx.x & 63u) * 1e-3f;
    const half8_t a = (half8_t)(_Float16)s, b = (half8_t)(_Float16)(1.0f - s);
    float4_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = (float4_t)0.0f;
    for (uint32_t i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[j], 0, 0, 0);
    }
    float4_t t = c[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) t += c[j];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = t[0] + t[1] + t[2] + t[3];
}

} // namespace

int launch_probe_read(const void *src, uint64_t n_bytes, uint32_t *sink, uint32_t n_wg, hipStream_t stream) {
    hipLaunchKernelGGL(k_probe_read, dim3(n_wg), dim3(256), 0, stream, (const u32x4_t *)src, n_bytes / 16u, sink);
    return hip_status(hipGetLastError());
}

int launch_probe_mfma(float *out, uint32_t n_wg, uint32_t iters, hipStream_t stream) {
    hipLaunchKernelGGL(k_probe_mfma, dim3(n_wg), dim3(256), 0, stream, out, iters, 0.25f);
    return hip_status(hipGetLastError());
}

} // namespace lfm
