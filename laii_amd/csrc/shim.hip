/*
 * shim.hip -- the extern "C" entry points of include/lfm_attn.h: argument
 * validation on the host, workspace management, and dispatch to the kernel
 * translation units.  No entry point enqueues work for a rejected call.
 */
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdio.h>
#include <string.h>
#include <vector>

#include "attn_index.h"
#include "kernels.h"
#include "lfm_attn.h"

namespace lfm {

static thread_local char g_last_error[256] = "";
static thread_local hipEvent_t g_prof_before = nullptr;
static thread_local hipEvent_t g_prof_after  = nullptr;
static thread_local const char *g_last_plan = "";

void note_plan(const char *name) { g_last_plan = name; }

void profile_events(hipEvent_t *before, hipEvent_t *after) {
    *before = g_prof_before;
    *after  = g_prof_after;
}

int hip_status(hipError_t e) {
    if (e == hipSuccess) return LFM_ATTN_OK;
    snprintf(g_last_error, sizeof g_last_error, "%s: %s", hipGetErrorName(e), hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? LFM_ATTN_E_NOMEM : LFM_ATTN_E_DEVICE;
}

namespace {
struct Workspace {
    void *ptr    = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::vector<Workspace> g_ws;
} // namespace

void *workspace(size_t bytes, hipStream_t stream, int *status) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) { *status = hip_status(e); return nullptr; }
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if ((size_t)dev >= g_ws.size()) g_ws.resize((size_t)dev + 1);
    Workspace &w = g_ws[(size_t)dev];
    if (w.bytes >= bytes) return w.ptr;
    if (w.ptr) {
        /* work already enqueued may still read the old buffer */
        e = hipStreamSynchronize(stream);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) { *status = hip_status(e); return nullptr; }
        (void)hipFree(w.ptr);
        w.ptr = nullptr;
        w.bytes = 0;
    }
    size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes + bytes / 4;
    e = hipMalloc(&w.ptr, want);
    if (e != hipSuccess) { w.ptr = nullptr; *status = hip_status(e); return nullptr; }
    w.bytes = want;
    return w.ptr;
}

/* Split partials of lfm_hip_gqa_f16_varlen_noalloc: one fixed array per
 * device, resolved to its device address once per device (the array's name
 * is a host-side stand-in: only the address from hipGetSymbolAddress may be
 * handed to kernels). */
static __device__ __align__(256) unsigned char scratch[LFM_ATTN_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mutex;
std::vector<void *> g_scratch_ptr;
} // namespace

static int noalloc_scratch(Scratch *out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if ((size_t)dev >= g_scratch_ptr.size()) g_scratch_ptr.resize((size_t)dev + 1, nullptr);
    if (!g_scratch_ptr[(size_t)dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e);
        if (!ptr) return LFM_ATTN_E_DEVICE;
        g_scratch_ptr[(size_t)dev] = ptr;
    }
    out->ptr   = g_scratch_ptr[(size_t)dev];
    out->bytes = LFM_ATTN_NOALLOC_SCRATCH_BYTES;
    return LFM_ATTN_OK;
}

} // namespace lfm

using lfm::AttnBatch;

static inline hipStream_t to_stream(lfm_attn_stream_t s) { return reinterpret_cast<hipStream_t>(s); }
static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0u; }
static inline bool prologue_form_ok(int f) { return f == LFM_PROLOGUE_FAST || f == LFM_PROLOGUE_TABLE; }

static int dispatch_f16(const AttnBatch &b, uint32_t keys_hint, hipStream_t stream,
                        const lfm::Scratch *sc = nullptr) {
    const bool fast = lfm::splitkv_supports(b) && aligned16(b.q) && aligned16(b.out) &&
                      (b.k_seq || (aligned16(b.k_base) && aligned16(b.v_base)));
    if (fast) return lfm::launch_splitkv(b, keys_hint, stream, sc);
    return lfm::launch_generic(b, false, stream);
}

extern "C" {

const char *lfm_attn_status_string(int status) {
    switch (status) {
    case LFM_ATTN_OK: return "ok";
    case LFM_ATTN_E_INVALID: return "invalid argument";
    case LFM_ATTN_E_RANGE: return "position out of range";
    case LFM_ATTN_E_UNSUPPORTED: return "unsupported shape";
    case LFM_ATTN_E_DEVICE: return "device error";
    case LFM_ATTN_E_NOMEM: return "out of device memory";
    case LFM_ATTN_E_IO: return "file could not be written";
    case LFM_ATTN_E_SCRATCH: return "split partials exceed the no-alloc scratch";
    default: return "unknown status";
    }
}

const char *lfm_attn_last_error(void) { return lfm::g_last_error; }

const char *lfm_attn_last_plan(void) { return lfm::g_last_plan; }

const char *lfm_attn_version(void) { return "lfm_attn 0.1 gfx950"; }

int lfm_attn_set_tuning(const char *plan, uint32_t waves, uint32_t chunk, uint32_t min_tiles,
                        uint32_t prefill_chain) {
    return lfm::set_tuning(plan, waves, chunk, min_tiles, prefill_chain);
}

int lfm_attn_plan_preview(uint32_t n_seq, uint32_t n_rows, uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                          uint32_t window_len, uint32_t keys_hint, int positions_on_device, int fused, uint32_t n_cus,
                          const char **plan, uint32_t out3[3]) {
    if (!plan || !out3 || n_seq == 0u || n_rows == 0u || n_head_q == 0u || n_head_kv == 0u ||
        n_head_q % n_head_kv != 0u || n_cus == 0u)
        return LFM_ATTN_E_INVALID;
    AttnBatch b;
    b.n_seq = n_seq;
    b.n_rows = n_rows;
    b.n_head_q = n_head_q;
    b.n_head_kv = n_head_kv;
    b.head_dim = head_dim;
    b.window = window_len;
    if (!lfm::splitkv_supports(b)) {
        *plan = "generic";
        out3[0] = out3[1] = out3[2] = 0u;
        return LFM_ATTN_OK;
    }
    const lfm::PlanChoice pc =
        lfm::choose_plan(b, keys_hint, positions_on_device != 0, fused != 0, n_cus, lfm::current_tuning());
    *plan   = lfm::plan_name(pc.kind);
    out3[0] = pc.waves;
    out3[1] = pc.kind == 'b' || pc.kind == 'd' ? 0u : pc.n_splits;
    out3[2] = pc.kind == 'b' || pc.kind == 'd' ? 0u : pc.chunk;
    return LFM_ATTN_OK;
}

int lfm_attn_prefill_plan_preview(uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint32_t window_len,
                                  uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim, uint32_t out4[4]) {
    if (!out4 || n_seq == 0u || n_tok == 0u || n_head_q == 0u || n_head_kv == 0u || n_head_q % n_head_kv != 0u)
        return LFM_ATTN_E_INVALID;
    if (!lfm::prefill_ext_supports(head_dim, n_head_q / n_head_kv)) return LFM_ATTN_E_UNSUPPORTED;
    const lfm::PrefillExtPlan pl = lfm::prefill_ext_plan(n_seq, n_tok, pos_0, window_len, n_head_q, n_head_kv);
    out4[0] = pl.tq;
    out4[1] = pl.chain;
    out4[2] = pl.n_light;
    out4[3] = pl.n_wg;
    return LFM_ATTN_OK;
}

int lfm_attn_profile_events(void *before, void *after) {
    if ((before == nullptr) != (after == nullptr)) return LFM_ATTN_E_INVALID;
    lfm::g_prof_before = reinterpret_cast<hipEvent_t>(before);
    lfm::g_prof_after  = reinterpret_cast<hipEvent_t>(after);
    return LFM_ATTN_OK;
}

int lfm_attn_device_count(int *count) {
    if (!count) return LFM_ATTN_E_INVALID;
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) { *count = 0; return LFM_ATTN_OK; }
    return lfm::hip_status(e);
}

int lfm_attn_set_device(int device) {
    const int st = lfm::hip_status(hipSetDevice(device));
    if (st != LFM_ATTN_OK) return st;
    /* resolve the no-alloc scratch of this device now, outside any graph
     * capture a caller may start later */
    lfm::Scratch sc;
    return lfm::noalloc_scratch(&sc);
}

int lfm_attn_dev_alloc(void **ptr, size_t bytes) {
    if (!ptr) return LFM_ATTN_E_INVALID;
    *ptr = nullptr;
    if (bytes == 0) return LFM_ATTN_OK;
    return lfm::hip_status(hipMalloc(ptr, bytes));
}

int lfm_attn_dev_free(void *ptr) { return ptr ? lfm::hip_status(hipFree(ptr)) : LFM_ATTN_OK; }

int lfm_attn_copy_h2d(void *dst, const void *src, size_t bytes, lfm_attn_stream_t stream) {
    if ((!dst || !src) && bytes) return LFM_ATTN_E_INVALID;
    if (!bytes) return LFM_ATTN_OK;
    return lfm::hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, to_stream(stream)));
}

int lfm_attn_copy_d2h(void *dst, const void *src, size_t bytes, lfm_attn_stream_t stream) {
    if ((!dst || !src) && bytes) return LFM_ATTN_E_INVALID;
    if (!bytes) return LFM_ATTN_OK;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, to_stream(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(to_stream(stream));
    return lfm::hip_status(e);
}

int lfm_attn_copy_d2d(void *dst, const void *src, size_t bytes, lfm_attn_stream_t stream) {
    if ((!dst || !src) && bytes) return LFM_ATTN_E_INVALID;
    if (!bytes) return LFM_ATTN_OK;
    return lfm::hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, to_stream(stream)));
}

int lfm_attn_memset(void *dst, int value, size_t bytes, lfm_attn_stream_t stream) {
    if (!dst && bytes) return LFM_ATTN_E_INVALID;
    if (!bytes) return LFM_ATTN_OK;
    return lfm::hip_status(hipMemsetAsync(dst, value, bytes, to_stream(stream)));
}

int lfm_attn_stream_sync(lfm_attn_stream_t stream) {
    return lfm::hip_status(hipStreamSynchronize(to_stream(stream)));
}

int lfm_attn_seg_plan(uint32_t abs_pos, uint32_t window_len, uint32_t cap, uint32_t out5[5]) {
    if (!out5) return LFM_ATTN_E_INVALID;
    if (window_len > 0u && (cap == 0u || window_len > cap)) return LFM_ATTN_E_INVALID;
    const lfm_seg_plan_t p = lfm_plan_row(abs_pos, window_len, cap);
    out5[0] = p.t_start;
    out5[1] = p.count;
    out5[2] = p.seg1_slot;
    out5[3] = p.seg1_len;
    out5[4] = p.seg2_len;
    return LFM_ATTN_OK;
}

uint32_t lfm_attn_slot_of(uint32_t p, uint32_t window_len, uint32_t cap) {
    if (window_len > 0u && cap == 0u) return 0u;
    return lfm_slot_of(p, window_len, cap);
}

/* ---- prologue ----------------------------------------------------------------- */
int lfm_hip_qk_norm_rope(float *vec, uint16_t *dst_f16, uint32_t n_heads, uint32_t head_dim,
                         const float *norm_w, float eps, const float *cos_lut,
                         const float *sin_lut, uint32_t pos, int prologue, lfm_attn_stream_t stream) {
    if (!vec || !cos_lut || !sin_lut || n_heads == 0u) return LFM_ATTN_E_INVALID;
    if (head_dim == 0u || (head_dim & 1u) || head_dim > 256u) return LFM_ATTN_E_INVALID;
    if (!prologue_form_ok(prologue)) return LFM_ATTN_E_INVALID;
    return lfm::launch_qk_norm_rope(vec, dst_f16, n_heads, head_dim, norm_w, eps, cos_lut, sin_lut,
                                    pos, prologue, to_stream(stream));
}

int lfm_hip_store_fp32_to_fp16(uint16_t *dst_f16, const float *src, uint32_t n,
                               lfm_attn_stream_t stream) {
    if (!dst_f16 || !src) return n ? LFM_ATTN_E_INVALID : LFM_ATTN_OK;
    if (n == 0u) return LFM_ATTN_OK;
    return lfm::launch_store_f16(dst_f16, src, n, to_stream(stream));
}

int lfm_hip_qkv_prologue(float *q, const float *k, const float *v, uint16_t *const *k_seq,
                         uint16_t *const *v_seq, const uint32_t *pos_0, uint32_t n_seq,
                         uint32_t n_rows, uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                         const float *q_norm_w, const float *k_norm_w, float eps,
                         const float *cos_lut, const float *sin_lut, uint32_t window_len,
                         uint32_t cap, int prologue, lfm_attn_stream_t stream) {
    if (!q || !k || !v || !k_seq || !v_seq || !pos_0 || !cos_lut || !sin_lut) return LFM_ATTN_E_INVALID;
    if (n_seq == 0u || n_rows == 0u || n_head_q == 0u || n_head_kv == 0u) return LFM_ATTN_E_INVALID;
    if (head_dim == 0u || (head_dim & 1u) || head_dim > 256u) return LFM_ATTN_E_INVALID;
    if (window_len > 0u && (cap == 0u || window_len > cap)) return LFM_ATTN_E_INVALID;
    if (!prologue_form_ok(prologue)) return LFM_ATTN_E_INVALID;
    return lfm::launch_qkv_prologue(q, k, v, k_seq, v_seq, pos_0, n_seq, n_rows, n_head_q, n_head_kv,
                                    head_dim, q_norm_w, k_norm_w, eps, cos_lut, sin_lut, window_len,
                                    cap, prologue, to_stream(stream));
}

/* ---- FNV-1a 64 of a device buffer ------------------------------------------- */
int lfm_hip_fnv1a64(const void *data, size_t n_bytes, uint64_t h_in, uint64_t *h_out, lfm_attn_stream_t stream) {
    if (!h_out) return LFM_ATTN_E_INVALID;
    if (n_bytes == 0u) {
        *h_out = h_in;
        return LFM_ATTN_OK;
    }
    if (!data || ((uintptr_t)data & 15u)) return LFM_ATTN_E_INVALID;
    const hipStream_t s = to_stream(stream);
    int st              = LFM_ATTN_OK;
    void *ws            = lfm::workspace(lfm::fnv1a64_workspace_bytes(n_bytes), s, &st);
    if (!ws) return st;
    if (lfm::launch_fnv1a64(data, n_bytes, h_in, ws, s) != 0) return lfm::hip_status(hipGetLastError());
    uint64_t acc = 0;
    hipError_t e = hipMemcpyAsync(&acc, ws, sizeof acc, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return lfm::hip_status(e);
    *h_out = lfm::fnv1a64_finish(h_in, n_bytes, acc);
    return LFM_ATTN_OK;
}

/* ---- achievable-peak probes ------------------------------------------------ */
int lfm_hip_probe_read(const void *src, uint64_t n_bytes, uint32_t *sink, uint32_t n_wg,
                       lfm_attn_stream_t stream) {
    if (!src || !sink || n_wg == 0u || n_bytes < 16u || ((uintptr_t)src & 15u)) return LFM_ATTN_E_INVALID;
    return lfm::launch_probe_read(src, n_bytes, sink, n_wg, to_stream(stream));
}

int lfm_hip_probe_mfma(float *out, uint32_t n_wg, uint32_t iters, lfm_attn_stream_t stream) {
    if (!out || n_wg == 0u || iters == 0u) return LFM_ATTN_E_INVALID;
    return lfm::launch_probe_mfma(out, n_wg, iters, to_stream(stream));
}

/* ---- projections beside the path ------------------------------------------- */
static inline bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1u)) == 0u; }

/* Weight types of the projections and the alignment their rows need (0: no
 * kernel): Q4_K and Q5_K blocks are 16-byte multiples, IQ4_XS 8, Q6_K,
 * Q4_0 and Q8_0 only 2. */
static inline uint32_t q_type_alignment(uint32_t type) {
    switch (type) {
    case 12u: case 13u: return 16u;
    case 23u: return 8u;
    case 14u: case 2u: case 8u: return 2u;
    default: return 0u;
    }
}

int lfm_hip_quantize_q8_K(const float *x, void *y_q8_K, uint32_t n_rows, uint32_t n_cols,
                          lfm_attn_stream_t stream) {
    if (n_rows == 0u || n_cols == 0u) return LFM_ATTN_OK;
    if (!x || !y_q8_K) return LFM_ATTN_E_INVALID;
    if (n_cols % 256u) return LFM_ATTN_E_UNSUPPORTED;
    if (!aligned(x, 4) || !aligned(y_q8_K, 4)) return LFM_ATTN_E_INVALID;
    return lfm::launch_quantize_q8_K(x, y_q8_K, n_rows, n_cols, to_stream(stream));
}

int lfm_hip_matmul_q4_K(float *out, const void *w_q4_K, uint32_t n_rows, uint32_t n_cols,
                        const void *x_q8_K, uint32_t n_tokens, lfm_attn_stream_t stream) {
    if (n_rows == 0u || n_tokens == 0u) return LFM_ATTN_OK;
    if (!out || !w_q4_K || !x_q8_K || n_cols == 0u) return LFM_ATTN_E_INVALID;
    if (n_cols % 256u) return LFM_ATTN_E_UNSUPPORTED;
    if (!aligned(w_q4_K, 16) || !aligned(x_q8_K, 4) || !aligned(out, 4)) return LFM_ATTN_E_INVALID;
    const uint32_t type = 12u;
    return lfm::launch_matmul_q(1u, &out, &w_q4_K, &type, &n_rows, n_cols, x_q8_K, n_tokens, to_stream(stream));
}

int lfm_hip_gqa_qkv_fused(float *q_out, float *k_out, float *v_out, float *g_out, const void *wq,
                          const void *wk, const void *wv, const void *wg, const uint32_t types[4],
                          uint32_t q_rows, uint32_t k_rows, uint32_t v_rows, uint32_t g_rows, uint32_t n_cols,
                          const void *x_q8_K, uint32_t n_tokens, lfm_attn_stream_t stream) {
    if (!types) return LFM_ATTN_E_INVALID;
    float *outs[4]       = {q_out, k_out, v_out, g_out};
    const void *ws[4]    = {wq, wk, wv, wg};
    const uint32_t rows[4] = {q_rows, k_rows, v_rows, g_out ? g_rows : 0u};
    if (n_tokens == 0u) return LFM_ATTN_OK;
    if (!x_q8_K || n_cols == 0u || !aligned(x_q8_K, 4)) return LFM_ATTN_E_INVALID;
    if (n_cols % 256u) return LFM_ATTN_E_UNSUPPORTED;
    for (int m = 0; m < 4; ++m) {
        if (rows[m] == 0u) continue;
        if (!outs[m] || !ws[m] || !aligned(outs[m], 4)) return LFM_ATTN_E_INVALID;
        const uint32_t need = q_type_alignment(types[m]);
        if (!need) return LFM_ATTN_E_UNSUPPORTED;
        if (!aligned(ws[m], need)) return LFM_ATTN_E_INVALID;
    }
    return lfm::launch_matmul_q(4u, outs, ws, types, rows, n_cols, x_q8_K, n_tokens, to_stream(stream));
}

int lfm_hip_matmul_prequant(float *out, const void *w, uint32_t w_type, uint32_t n_rows, uint32_t n_cols,
                            const void *x_q8_K, uint32_t n_tokens, lfm_attn_stream_t stream) {
    if (n_rows == 0u || n_tokens == 0u) return LFM_ATTN_OK;
    if (!out || !w || !x_q8_K || n_cols == 0u || !aligned(x_q8_K, 4) || !aligned(out, 4)) return LFM_ATTN_E_INVALID;
    const uint32_t need = q_type_alignment(w_type);
    if (!need || n_cols % 256u) return LFM_ATTN_E_UNSUPPORTED;
    if (!aligned(w, need)) return LFM_ATTN_E_INVALID;
    return lfm::launch_matmul_q(1u, &out, &w, &w_type, &n_rows, n_cols, x_q8_K, n_tokens, to_stream(stream));
}

/* ---- attention -------------------------------------------------------------- */
int lfm_hip_online_gqa_f16(const float *q, const uint16_t *k_cache_f16,
                           const uint16_t *v_cache_f16, float *xb_out, uint32_t n_head_q,
                           uint32_t kv_mul, uint32_t kv_dim, uint32_t pos, float scale,
                           lfm_attn_stream_t stream) {
    if (!q || !k_cache_f16 || !v_cache_f16 || !xb_out) return LFM_ATTN_E_INVALID;
    if (n_head_q == 0u || kv_mul == 0u || n_head_q % kv_mul != 0u) return LFM_ATTN_E_INVALID;
    if (kv_dim != (n_head_q / kv_mul) * 64u) return LFM_ATTN_E_INVALID;
    if (pos >= 0x7FFFFFFFu) return LFM_ATTN_E_RANGE;
    AttnBatch b;
    b.q = q;
    b.k_base = k_cache_f16;
    b.v_base = v_cache_f16;
    b.pos0_host = pos;
    b.out = xb_out;
    b.out_dims = 64u;
    b.n_head_q = n_head_q;
    b.n_head_kv = n_head_q / kv_mul;
    b.head_dim = 64u;
    b.scale = scale;
    return dispatch_f16(b, pos + 1u, to_stream(stream));
}

int lfm_hip_gqa_heads(const float *q, const float *k_cache, const float *v_cache,
                      const uint16_t *k_cache_f16, const uint16_t *v_cache_f16, float *xb,
                      uint32_t n_head_q, uint32_t kv_mul, uint32_t head_dim, uint32_t kv_dim,
                      uint32_t max_seq_len, uint32_t pos, float scale, lfm_attn_stream_t stream) {
    const bool f16 = k_cache_f16 && v_cache_f16;
    if (!q || !xb || (!f16 && (!k_cache || !v_cache))) return LFM_ATTN_E_INVALID;
    if (n_head_q == 0u || kv_mul == 0u || n_head_q % kv_mul != 0u) return LFM_ATTN_E_INVALID;
    if (head_dim == 0u || head_dim % 8u != 0u || head_dim > 256u) return LFM_ATTN_E_INVALID;
    if (kv_dim != (n_head_q / kv_mul) * head_dim) return LFM_ATTN_E_INVALID;
    if (pos >= max_seq_len || pos >= 0x7FFFFFFFu) return LFM_ATTN_E_RANGE;
    AttnBatch b;
    b.q = q;
    b.pos0_host = pos;
    b.out = xb;
    b.n_head_q = n_head_q;
    b.n_head_kv = n_head_q / kv_mul;
    b.head_dim = head_dim;
    b.scale = scale;
    if (f16) {
        /* tools/lfm2_threadpool.c:783: the fp16 branch writes n_vec*8 dims */
        b.out_dims = head_dim <= 64u ? head_dim : 64u;
        b.k_base = k_cache_f16;
        b.v_base = v_cache_f16;
        return dispatch_f16(b, pos + 1u, to_stream(stream));
    }
    b.out_dims = head_dim;
    b.k_base = k_cache;
    b.v_base = v_cache;
    return lfm::launch_generic(b, true, to_stream(stream));
}

int lfm_hip_lfm3_online_gqa_f16_dispatch(const float *q_batch, const float *gate_sig,
                                         const uint16_t *k_cache_f16,
                                         const uint16_t *v_cache_f16, float *xb_out, uint32_t B,
                                         uint32_t pos_0, uint32_t window_len, uint32_t swa_cap,
                                         uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim,
                                         lfm_attn_stream_t stream) {
    if (!q_batch || !k_cache_f16 || !v_cache_f16 || !xb_out) return LFM_ATTN_E_INVALID;
    if (B == 0u || n_head_q == 0u || n_head_kv == 0u || n_head_q % n_head_kv != 0u)
        return LFM_ATTN_E_INVALID;
    if (head_dim == 0u || head_dim % 8u != 0u || head_dim > 256u) return LFM_ATTN_E_INVALID;
    if (window_len > 0u && (swa_cap == 0u || window_len > swa_cap)) return LFM_ATTN_E_INVALID;
    if (lfm_check_rows(pos_0, B, window_len, swa_cap) != 0 || pos_0 >= 0x7FFFFFFFu)
        return LFM_ATTN_E_RANGE;
    AttnBatch b;
    b.q = q_batch;
    b.gate = gate_sig;
    b.k_base = k_cache_f16;
    b.v_base = v_cache_f16;
    b.pos0_host = pos_0;
    b.out = xb_out;
    b.out_dims = head_dim;
    b.n_rows = B;
    b.n_head_q = n_head_q;
    b.n_head_kv = n_head_kv;
    b.head_dim = head_dim;
    b.window = window_len;
    b.cap = swa_cap;
    b.scale = 1.0f / sqrtf((float)head_dim);
    const uint32_t max_keys = window_len ? window_len : pos_0 + B;
    return dispatch_f16(b, max_keys, to_stream(stream));
}

static int varlen_call(const float *q, const float *gate, int gate_is_logit, const uint16_t *const *k_seq,
                       const uint16_t *const *v_seq, const uint32_t *pos_0, float *out, uint32_t n_seq,
                       uint32_t n_rows, uint32_t keys_hint, uint32_t n_head_q, uint32_t n_head_kv,
                       uint32_t head_dim, uint32_t window_len, uint32_t cap, float scale,
                       lfm_attn_stream_t stream, bool noalloc) {
    if (!q || !k_seq || !v_seq || !pos_0 || !out) return LFM_ATTN_E_INVALID;
    if (n_seq == 0u || n_rows == 0u || n_head_q == 0u || n_head_kv == 0u ||
        n_head_q % n_head_kv != 0u)
        return LFM_ATTN_E_INVALID;
    if (n_seq > 65535u || n_head_kv > 65535u) return LFM_ATTN_E_INVALID;
    if (head_dim == 0u || head_dim % 8u != 0u || head_dim > 256u) return LFM_ATTN_E_INVALID;
    if (window_len > 0u && (cap == 0u || window_len > cap)) return LFM_ATTN_E_INVALID;
    AttnBatch b;
    b.q = q;
    b.gate = gate;
    b.gate_is_logit = gate_is_logit;
    b.k_seq = reinterpret_cast<const void *const *>(k_seq);
    b.v_seq = reinterpret_cast<const void *const *>(v_seq);
    b.pos0_dev = pos_0;
    b.out = out;
    b.out_dims = head_dim;
    b.n_seq = n_seq;
    b.n_rows = n_rows;
    b.n_head_q = n_head_q;
    b.n_head_kv = n_head_kv;
    b.head_dim = head_dim;
    b.window = window_len;
    b.cap = cap;
    b.scale = scale;
    if (!noalloc) return dispatch_f16(b, keys_hint, to_stream(stream));
    lfm::Scratch sc;
    const int st = lfm::noalloc_scratch(&sc);
    if (st != LFM_ATTN_OK) return st;
    return dispatch_f16(b, keys_hint, to_stream(stream), &sc);
}

int lfm_hip_gqa_f16_varlen(const float *q, const float *gate, int gate_is_logit,
                           const uint16_t *const *k_seq, const uint16_t *const *v_seq,
                           const uint32_t *pos_0, float *out, uint32_t n_seq, uint32_t n_rows,
                           uint32_t keys_hint, uint32_t n_head_q, uint32_t n_head_kv,
                           uint32_t head_dim, uint32_t window_len, uint32_t cap, float scale,
                           lfm_attn_stream_t stream) {
    return varlen_call(q, gate, gate_is_logit, k_seq, v_seq, pos_0, out, n_seq, n_rows, keys_hint, n_head_q,
                       n_head_kv, head_dim, window_len, cap, scale, stream, false);
}

int lfm_hip_gqa_f16_varlen_noalloc(const float *q, const float *gate, int gate_is_logit,
                                   const uint16_t *const *k_seq, const uint16_t *const *v_seq,
                                   const uint32_t *pos_0, float *out, uint32_t n_seq, uint32_t n_rows,
                                   uint32_t keys_hint, uint32_t n_head_q, uint32_t n_head_kv,
                                   uint32_t head_dim, uint32_t window_len, uint32_t cap, float scale,
                                   lfm_attn_stream_t stream) {
    return varlen_call(q, gate, gate_is_logit, k_seq, v_seq, pos_0, out, n_seq, n_rows, keys_hint, n_head_q,
                       n_head_kv, head_dim, window_len, cap, scale, stream, true);
}

int lfm_hip_gen1_gqa_step(float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                          float *k_cache, float *v_cache, float *attn_out, uint32_t pos, uint32_t max_seq,
                          uint32_t n_heads_q, uint32_t n_heads_kv, uint32_t head_dim, float eps,
                          const float *cos_row, const float *sin_row, lfm_attn_stream_t stream) {
    if (!q || !k || !v || !k_cache || !v_cache || !attn_out || !cos_row || !sin_row) return LFM_ATTN_E_INVALID;
    if (n_heads_q == 0u || n_heads_kv == 0u || n_heads_q % n_heads_kv != 0u) return LFM_ATTN_E_INVALID;
    if (head_dim == 0u || head_dim % 8u != 0u || head_dim > 256u) return LFM_ATTN_E_INVALID;
    if (pos >= max_seq || pos >= 0x7FFFFFFFu) return LFM_ATTN_E_RANGE;
    const hipStream_t st = to_stream(stream);
    const int r = lfm::launch_gen1_prologue(q, k, v, k_cache, v_cache, q_norm, k_norm, eps, cos_row, sin_row, pos,
                                            n_heads_q, n_heads_kv, head_dim, st);
    if (r != LFM_ATTN_OK) return r;
    AttnBatch b;
    b.q = q;
    b.k_base = k_cache;
    b.v_base = v_cache;
    b.pos0_host = pos;
    b.out = attn_out;
    b.out_dims = head_dim;
    b.n_head_q = n_heads_q;
    b.n_head_kv = n_heads_kv;
    b.head_dim = head_dim;
    b.scale = 1.0f / sqrtf((float)head_dim);
    return lfm::launch_generic(b, true, st);
}

int lfm_hip_gqa_f16_step(const float *q, const float *k, const float *v, const float *gate, int gate_is_logit,
                         uint16_t *const *k_seq, uint16_t *const *v_seq, const uint32_t *pos_0, float *out,
                         uint32_t n_seq, uint32_t n_rows, uint32_t keys_hint, uint32_t n_head_q,
                         uint32_t n_head_kv, uint32_t head_dim, uint32_t window_len, uint32_t cap, float scale,
                         const float *q_norm_w, const float *k_norm_w, float eps, const float *cos_lut,
                         const float *sin_lut, int prologue, lfm_attn_stream_t stream) {
    if (!q || !k || !v || !k_seq || !v_seq || !pos_0 || !out || !cos_lut || !sin_lut) return LFM_ATTN_E_INVALID;
    if (!prologue_form_ok(prologue)) return LFM_ATTN_E_INVALID;
    if (n_seq == 0u || n_rows == 0u || n_head_q == 0u || n_head_kv == 0u || n_head_q % n_head_kv != 0u)
        return LFM_ATTN_E_INVALID;
    if (n_seq > 65535u || n_head_kv > 65535u) return LFM_ATTN_E_INVALID;
    if (head_dim == 0u || head_dim % 8u != 0u || head_dim > 256u) return LFM_ATTN_E_INVALID;
    if (window_len > 0u && (cap == 0u || window_len > cap)) return LFM_ATTN_E_INVALID;
    /* every row's window must survive the later rows' ring writes */
    if (window_len > 0u && (uint64_t)window_len + n_rows - 1u > cap) return LFM_ATTN_E_INVALID;
    AttnBatch b;
    b.q = q;
    b.gate = gate;
    b.gate_is_logit = gate_is_logit;
    b.k_seq = reinterpret_cast<const void *const *>(k_seq);
    b.v_seq = reinterpret_cast<const void *const *>(v_seq);
    b.pos0_dev = pos_0;
    b.out = out;
    b.out_dims = head_dim;
    b.n_seq = n_seq;
    b.n_rows = n_rows;
    b.n_head_q = n_head_q;
    b.n_head_kv = n_head_kv;
    b.head_dim = head_dim;
    b.window = window_len;
    b.cap = cap;
    b.scale = scale;
    const hipStream_t st = to_stream(stream);
    const bool fused = lfm::splitkv_supports(b) && aligned16(q) && aligned16(out) && aligned16(k) && aligned16(v) &&
                       aligned16(cos_lut) && aligned16(sin_lut) && (!q_norm_w || aligned16(q_norm_w)) &&
                       (!k_norm_w || aligned16(k_norm_w));
    if (fused) {
        b.k_new = k;
        b.v_new = v;
        b.q_norm_w = q_norm_w;
        b.k_norm_w = k_norm_w;
        b.cos_lut = cos_lut;
        b.sin_lut = sin_lut;
        b.eps = eps;
        b.prologue = prologue;
        return lfm::launch_splitkv(b, keys_hint, st);
    }
    /* shapes the split-KV kernel does not take: the prologue on a copy of q
     * (q stays as passed), then the generic kernel */
    const size_t q_bytes = (size_t)n_seq * n_rows * n_head_q * head_dim * sizeof(float);
    int ws_st = LFM_ATTN_OK;
    float *qw = static_cast<float *>(lfm::workspace(q_bytes, st, &ws_st));
    if (!qw) return ws_st;
    int r = lfm::hip_status(hipMemcpyAsync(qw, q, q_bytes, hipMemcpyDeviceToDevice, st));
    if (r != LFM_ATTN_OK) return r;
    r = lfm::launch_qkv_prologue(qw, k, v, k_seq, v_seq, pos_0, n_seq, n_rows, n_head_q, n_head_kv, head_dim,
                                 q_norm_w, k_norm_w, eps, cos_lut, sin_lut, window_len, cap, prologue, st);
    if (r != LFM_ATTN_OK) return r;
    b.q = qw;
    return lfm::launch_generic(b, false, st);
}

int lfm_hip_prefill_f16(const float *q, const uint16_t *k, const uint16_t *v, float *out,
                        uint32_t n_seq, uint32_t n_tok, uint32_t pos_0, uint64_t kv_seq_stride,
                        uint32_t n_head_q, uint32_t n_head_kv, uint32_t head_dim, float scale,
                        lfm_attn_stream_t stream) {
    if (!q || !k || !v || !out) return LFM_ATTN_E_INVALID;
    if (n_seq == 0u || n_tok == 0u || n_head_q == 0u || n_head_kv == 0u ||
        n_head_q % n_head_kv != 0u)
        return LFM_ATTN_E_INVALID;
    if (n_seq > 65535u || n_head_kv > 65535u) return LFM_ATTN_E_INVALID;
    if ((uint64_t)pos_0 + n_tok > 0x7FFFFFFFull) return LFM_ATTN_E_RANGE;
    if (n_seq > 1u && kv_seq_stride < ((uint64_t)pos_0 + n_tok) * n_head_kv * head_dim)
        return LFM_ATTN_E_INVALID; /* sequences would overlap */
    if (!lfm::prefill_supports(head_dim, n_head_q / n_head_kv)) return LFM_ATTN_E_UNSUPPORTED;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || (kv_seq_stride % 8u))
        return LFM_ATTN_E_INVALID;
    return lfm::launch_prefill(q, k, v, out, n_seq, n_tok, pos_0, kv_seq_stride, n_head_q,
                               n_head_kv, head_dim, scale, to_stream(stream));
}

int lfm_hip_lfm3_prefill_f16(const float *q, const uint16_t *k, const uint16_t *v, const float *gate,
                             int gate_is_logit, float *out, uint32_t n_seq, uint32_t n_tok, uint32_t pos_0,
                             uint32_t kv_pos0, uint64_t kv_seq_stride, uint32_t window_len, uint32_t n_head_q,
                             uint32_t n_head_kv, uint32_t head_dim, float scale, lfm_attn_stream_t stream) {
    if (!q || !k || !v || !out) return LFM_ATTN_E_INVALID;
    if (n_seq == 0u || n_tok == 0u || n_head_q == 0u || n_head_kv == 0u || n_head_q % n_head_kv != 0u)
        return LFM_ATTN_E_INVALID;
    if (n_seq > 65535u || n_head_kv > 65535u) return LFM_ATTN_E_INVALID;
    if ((uint64_t)pos_0 + n_tok > 0x7FFFFFFFull) return LFM_ATTN_E_RANGE;
    /* every key a row attends must be in the buffer: kv_pos0 <= t_start(pos_0) */
    const uint32_t t_first = (window_len > 0u && pos_0 + 1u > window_len) ? pos_0 + 1u - window_len : 0u;
    if (kv_pos0 > t_first) return LFM_ATTN_E_INVALID;
    const uint64_t rows = (uint64_t)pos_0 + n_tok - kv_pos0;
    if (n_seq > 1u && kv_seq_stride < rows * n_head_kv * head_dim)
        return LFM_ATTN_E_INVALID; /* sequences would overlap */
    if (!lfm::prefill_ext_supports(head_dim, n_head_q / n_head_kv)) return LFM_ATTN_E_UNSUPPORTED;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || (kv_seq_stride % 8u))
        return LFM_ATTN_E_INVALID;
    return lfm::launch_prefill_ext(q, k, v, gate, gate_is_logit, out, n_seq, n_tok, pos_0, kv_pos0,
                                   kv_seq_stride, window_len, n_head_q, n_head_kv, head_dim, scale,
                                   to_stream(stream));
}

/* ---- attention-sink eviction ------------------------------------------- */

static inline int shift_caches_ok(uint16_t *const *k_caches, uint16_t *const *v_caches,
                                  const uint32_t *n_head_kv, uint32_t n_layers) {
    if (!k_caches || !v_caches || !n_head_kv) return 0;
    for (uint32_t l = 0; l < n_layers; ++l)
        if ((k_caches[l] && !aligned16(k_caches[l])) || (v_caches[l] && !aligned16(v_caches[l])))
            return 0;
    return 1;
}

int lfm_hip_kv_cache_shift_sinks(uint16_t *const *k_caches, uint16_t *const *v_caches,
                                 uint32_t n_layers, const uint32_t *n_head_kv, uint32_t head_dim,
                                 const float *cos_lut, const float *sin_lut, uint32_t lut_rows,
                                 uint32_t *inout_pos, uint32_t n_sink, uint32_t n_discard,
                                 lfm_attn_stream_t stream) {
    if (!inout_pos) return LFM_ATTN_E_INVALID;
    const uint32_t cur = *inout_pos;
    /* tools/lfm2_runtime_features.c:752-758: no-op cases keep the position */
    if (n_discard == 0u || (uint64_t)cur <= (uint64_t)n_sink + n_discard) return LFM_ATTN_OK;
    if (head_dim != 64u) return LFM_ATTN_OK;
    if (!shift_caches_ok(k_caches, v_caches, n_head_kv, n_layers) || !cos_lut || !sin_lut)
        return LFM_ATTN_E_INVALID;
    if (n_discard >= lut_rows) return LFM_ATTN_E_RANGE;
    const uint32_t n_keep = cur - n_sink - n_discard;
    const hipStream_t st = to_stream(stream);
    for (uint32_t l = 0; l < n_layers; ++l) {
        if (!k_caches[l] || !v_caches[l] || n_head_kv[l] == 0u) continue; /* ShortConv layer */
        const int r = lfm::launch_kv_shift(k_caches[l], v_caches[l], n_head_kv[l] * 64u, 64u, n_sink,
                                           n_keep, n_discard, cos_lut + (size_t)n_discard * 32u,
                                           sin_lut + (size_t)n_discard * 32u, st);
        if (r != LFM_ATTN_OK) return r;
    }
    *inout_pos = n_sink + n_keep;
    return LFM_ATTN_OK;
}

int lfm_hip_lfm3_kv_cache_shift_sinks(uint16_t *const *k_caches, uint16_t *const *v_caches,
                                      uint32_t n_layers, const uint32_t *n_head_kv,
                                      const uint8_t *layer_kind, uint32_t head_dim,
                                      const float *cos_full, const float *sin_full,
                                      uint32_t full_rows, const float *cos_swa,
                                      const float *sin_swa, uint32_t swa_rows,
                                      uint32_t sliding_window, uint32_t swa_cap,
                                      uint32_t *inout_pos, uint32_t n_sink, uint32_t n_discard,
                                      lfm_attn_stream_t stream) {
    if (!inout_pos || !cos_full || !sin_full || !cos_swa || !sin_swa) return LFM_ATTN_E_INVALID;
    const uint32_t cur = *inout_pos;
    /* tools/lfm2_runtime_features.c:1066-1073: no-op cases keep the position */
    if (n_discard == 0u || (uint64_t)cur <= (uint64_t)n_sink + n_discard) return LFM_ATTN_OK;
    if (n_discard >= full_rows || n_discard >= swa_rows) return LFM_ATTN_OK;
    if (head_dim % 2u != 0u) return LFM_ATTN_OK;
    if (head_dim % 16u != 0u || head_dim > 256u) return LFM_ATTN_E_UNSUPPORTED;
    if (!layer_kind || !shift_caches_ok(k_caches, v_caches, n_head_kv, n_layers))
        return LFM_ATTN_E_INVALID;
    const uint32_t half    = head_dim / 2u;
    const uint32_t n_keep  = cur - (n_sink + n_discard);
    const uint32_t new_pos = n_sink + n_keep;
    const uint32_t swa_win = sliding_window > 0u ? sliding_window : 256u;
    const uint32_t cap     = swa_cap > 0u ? swa_cap : swa_win + 8u;
    if (cap < swa_win) return LFM_ATTN_E_INVALID;
    const hipStream_t st = to_stream(stream);
    /* :1101-1135: an SWA layer re-slots the window [new_pos - window,
     * new_pos) through a staging area.  Every layer is checked, and the
     * largest stage reserved, before any layer is touched: a failure leaves
     * every cache as it was. */
    const uint32_t t0      = new_pos > swa_win ? new_pos - swa_win : 0u;
    const uint32_t n_valid = new_pos - t0;
    size_t stage_elems     = 0;
    for (uint32_t l = 0; l < n_layers; ++l) {
        if (layer_kind[l] == 0u || !k_caches[l] || !v_caches[l] || n_head_kv[l] == 0u) continue;
        if ((uint64_t)n_head_kv[l] * head_dim > 0xFFFFFFFFull) return LFM_ATTN_E_INVALID;
        const size_t e = (size_t)2u * n_valid * n_head_kv[l] * head_dim;
        if (layer_kind[l] == 2u && e > stage_elems) stage_elems = e;
    }
    uint16_t *stage = nullptr;
    if (stage_elems) {
        int ws_st = LFM_ATTN_OK;
        stage = (uint16_t *)lfm::workspace(stage_elems * sizeof(uint16_t), st, &ws_st);
        if (!stage) return ws_st;
    }
    for (uint32_t l = 0; l < n_layers; ++l) {
        if (layer_kind[l] == 0u || !k_caches[l] || !v_caches[l] || n_head_kv[l] == 0u) continue;
        const uint32_t kv_dim = n_head_kv[l] * head_dim;
        int r;
        if (layer_kind[l] == 2u) {
            r = lfm::launch_kv_swa_repack(k_caches[l], v_caches[l], kv_dim, head_dim, cap, t0, n_valid,
                                          n_sink, n_discard, cos_swa + (size_t)n_discard * half,
                                          sin_swa + (size_t)n_discard * half, stage,
                                          stage + (size_t)n_valid * kv_dim, st);
        } else {
            r = lfm::launch_kv_shift(k_caches[l], v_caches[l], kv_dim, head_dim, n_sink, n_keep,
                                     n_discard, cos_full + (size_t)n_discard * half,
                                     sin_full + (size_t)n_discard * half, st);
        }
        if (r != LFM_ATTN_OK) return r;
    }
    *inout_pos = new_pos;
    return LFM_ATTN_OK;
}

} /* extern "C" */
