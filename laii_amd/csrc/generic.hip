/*
 * generic.hip -- one wave64 per (query head, row, sequence); any head_dim with
 * head_dim % 8 == 0 and head_dim <= 256, fp16 or fp32 caches.
 *
 * Serves the shapes the MFMA split-KV kernel does not take: the FP32 two-pass
 * branch of lfm2_gqa_heads_worker_task (tools/lfm2_threadpool.c:887-928), the
 * Gen-1 FP32 cache (src/lfm_forward.c:204-244), and head dims other than 64
 * and 128.  Keys are visited one at a time in the order of the reference's
 * segment walk (tools/lfm3_engine.c:1103-1114) with the reference's per-key
 * recurrence (tools/lfm3_engine.c:1068-1089): a larger score rescales the
 * running sums by expf(m - s) (0 on the first key), a smaller one adds
 * expf(s - m).  The two-pass FP32 softmax of the reference computes the same
 * function; only the rounding differs.  Lane j owns dims j, j+64, j+128, j+192.
 */
#include <hip/hip_runtime.h>

#include "attn_index.h"
#include "kernels.h"
#include "lfm_attn.h"

namespace lfm {
namespace {

struct GenericParams {
    const float *q;
    const float *gate;
    const void *k_base;
    const void *v_base;
    const void *const *k_seq;
    const void *const *v_seq;
    uint64_t seq_stride;
    const uint32_t *pos0_dev;
    float *out;
    uint32_t pos0_host, n_rows, n_head_q, n_head_kv, head_dim, window, cap, out_dims;
    int gate_is_logit;
    float scale;
};

__device__ __forceinline__ float load_kv(const uint16_t *p, uint32_t i) {
    return (float)__builtin_bit_cast(_Float16, p[i]);
}
__device__ __forceinline__ float load_kv(const float *p, uint32_t i) { return p[i]; }

__device__ __forceinline__ float wave_sum_uniform(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
    /* every lane continues with lane 0's bits so branches stay uniform */
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

template <typename KV>
__global__ __launch_bounds__(64) void k_generic(const GenericParams G) {
    const uint32_t h = blockIdx.x, r = blockIdx.y, s = blockIdx.z;
    const uint32_t lane = threadIdx.x;
    const uint32_t hd   = G.head_dim;
    const uint32_t kv_mul = G.n_head_q / G.n_head_kv;
    const uint32_t pos0 = G.pos0_dev ? G.pos0_dev[s] : G.pos0_host;
    const lfm_seg_plan_t pl = lfm_plan_row(pos0 + r, G.window, G.cap);

    const KV *kc = G.k_seq ? static_cast<const KV *>(G.k_seq[s])
                           : static_cast<const KV *>(G.k_base) + (size_t)s * G.seq_stride;
    const KV *vc = G.v_seq ? static_cast<const KV *>(G.v_seq[s])
                           : static_cast<const KV *>(G.v_base) + (size_t)s * G.seq_stride;
    const size_t row = (size_t)G.n_head_kv * hd;
    kc += (size_t)(h / kv_mul) * hd;
    vc += (size_t)(h / kv_mul) * hd;

    const size_t orow = ((size_t)s * G.n_rows + r) * G.n_head_q + h;
    float qv[4], o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = lane + 64u * j;
        qv[j] = d < hd ? G.q[orow * hd + d] : 0.0f;
        o[j]  = 0.0f;
    }
    float m = -1e30f, l = 0.0f;
    for (uint32_t t = 0; t < pl.count; ++t) {
        const uint32_t slot = (t < pl.seg1_len) ? pl.seg1_slot + t : t - pl.seg1_len;
        const KV *kt = kc + (size_t)slot * row;
        const KV *vt = vc + (size_t)slot * row;
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = lane + 64u * j;
            if (d < hd) part += qv[j] * load_kv(kt, d);
        }
        const float score = wave_sum_uniform(part) * G.scale;
        if (score > m) {
            const float alpha = (m <= -1e29f) ? 0.0f : expf(m - score);
            l = l * alpha + 1.0f;
            m = score;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t d = lane + 64u * j;
                if (d < hd) o[j] = o[j] * alpha + load_kv(vt, d);
            }
        } else {
            const float beta = expf(score - m);
            l += beta;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t d = lane + 64u * j;
                if (d < hd) o[j] += beta * load_kv(vt, d);
            }
        }
    }
    float gv = 1.0f;
    if (G.gate) {
        gv = G.gate[orow];
        if (G.gate_is_logit) gv = 1.0f / (1.0f + expf(-gv));
    }
    const float inv = (l > 0.0f) ? gv / l : 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = lane + 64u * j;
        if (d < G.out_dims) G.out[orow * hd + d] = o[j] * inv;
    }
}

} // namespace

int launch_generic(const AttnBatch &b, bool kv_f32, hipStream_t stream) {
    note_plan("generic");
    GenericParams G{};
    G.q             = b.q;
    G.gate          = b.gate;
    G.gate_is_logit = b.gate_is_logit;
    G.k_base        = b.k_base;
    G.v_base        = b.v_base;
    G.k_seq         = b.k_seq;
    G.v_seq         = b.v_seq;
    G.seq_stride    = b.seq_stride;
    G.pos0_dev      = b.pos0_dev;
    G.pos0_host     = b.pos0_host;
    G.out           = b.out;
    G.n_rows        = b.n_rows;
    G.n_head_q      = b.n_head_q;
    G.n_head_kv     = b.n_head_kv;
    G.head_dim      = b.head_dim;
    G.window        = b.window;
    G.cap           = b.cap;
    G.out_dims      = b.out_dims;
    G.scale         = b.scale;
    dim3 grid(b.n_head_q, b.n_rows, b.n_seq);
    if (kv_f32) hipLaunchKernelGGL(k_generic<float>, grid, dim3(64), 0, stream, G);
    else hipLaunchKernelGGL(k_generic<uint16_t>, grid, dim3(64), 0, stream, G);
    return hip_status(hipGetLastError());
}

} // namespace lfm
