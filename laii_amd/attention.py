"""Python mirror of the reference's attention dispatch interface, running on
the MI355X kernels through the C-ABI.

Function names and argument meaning follow the reference task contexts:
  online_gqa_f16                 OnlineGQATaskCtx        tools/lfm2_kernels_fast.c:685-697
  gqa_heads                      GQAAttnTaskCtx          tools/lfm2_threadpool.c:746-762
  lfm3_online_gqa_f16_dispatch   lfm3_online_gqa_f16_dispatch tools/lfm3_engine.c:1155-1168
  qk_norm_rope                   lfm2/lfm3_qk_norm_rope_* tools/lfm2_kernels_fast.c:403-547,
                                                          tools/lfm3_engine.c:463-666
  rope_lut_lfm2 / rope_lut_lfm3  lfm2_rope_lut_init / lfm3_rope_lut_init
  rope_table_lfm2                the float-angle table of lfm2_state_init /
                                 lfm2_batch_state_init (prologue=PROLOGUE_TABLE)
Tensors are DeviceArray objects (device memory) or raw device addresses (int).
Every call raises LfmAttnError on a non-zero status; nothing falls back to
the CPU.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence, Union

import numpy as np

from ._lib import PROLOGUE_FAST, PROLOGUE_TABLE, CacheModelC, Geom, check, load

Ptr = Union["DeviceArray", int, None]


def device_count() -> int:
    n = C.c_int(0)
    check(load().lfm_attn_device_count(C.byref(n)), "lfm_attn_device_count")
    return int(n.value)


def require_gpu() -> None:
    if device_count() < 1:
        raise RuntimeError("no HIP device visible: the attention path runs only on the GPU")


class DeviceArray:
    """A device allocation with numpy upload/download (no torch involved)."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(x) for x in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p(0)
        check(load().lfm_attn_dev_alloc(C.byref(p), self.nbytes), "lfm_attn_dev_alloc")
        self.ptr = int(p.value or 0)

    @classmethod
    def from_numpy(cls, arr: np.ndarray, stream=None) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = cls(arr.shape, arr.dtype)
        d.upload(arr, stream)
        return d

    @classmethod
    def zeros(cls, shape, dtype) -> "DeviceArray":
        d = cls(shape, dtype)
        check(load().lfm_attn_memset(d.ptr, 0, d.nbytes, None), "lfm_attn_memset")
        return d

    def upload(self, arr: np.ndarray, stream=None) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        assert arr.nbytes == self.nbytes, (arr.nbytes, self.nbytes)
        check(load().lfm_attn_copy_h2d(self.ptr, arr.ctypes.data, self.nbytes, stream),
              "lfm_attn_copy_h2d")
        if stream is None:
            check(load().lfm_attn_stream_sync(None), "lfm_attn_stream_sync")

    def numpy(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(load().lfm_attn_copy_d2h(out.ctypes.data, self.ptr, self.nbytes, stream),
              "lfm_attn_copy_d2h")
        return out

    def free(self) -> None:
        if getattr(self, "ptr", 0):
            load().lfm_attn_dev_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __int__(self) -> int:
        return self.ptr


def _p(x: Ptr) -> Optional[int]:
    if x is None:
        return None
    return int(x)


def sync(stream=None) -> None:
    check(load().lfm_attn_stream_sync(stream), "lfm_attn_stream_sync")


def seg_plan(abs_pos: int, window_len: int, cap: int):
    out = (C.c_uint32 * 5)()
    check(load().lfm_attn_seg_plan(abs_pos, window_len, cap, out), "lfm_attn_seg_plan")
    return tuple(int(x) for x in out)


def slot_of(p: int, window_len: int, cap: int) -> int:
    return int(load().lfm_attn_slot_of(p, window_len, cap))


def rope_lut_lfm2(max_seq: int, head_dim: int, freq_base: float):
    c = np.empty((max_seq, head_dim // 2), np.float32)
    s = np.empty_like(c)
    check(load().lfm_attn_rope_lut_lfm2(c.ctypes.data, s.ctypes.data, max_seq, head_dim, freq_base),
          "lfm_attn_rope_lut_lfm2")
    return c, s


def rope_lut_lfm3(max_seq: int, head_dim: int, rope_dim: int, freq_base: float,
                  rope_freqs: Optional[np.ndarray] = None):
    c = np.empty((max_seq, head_dim // 2), np.float32)
    s = np.empty_like(c)
    rf = None if rope_freqs is None else np.ascontiguousarray(rope_freqs, np.float32)
    check(load().lfm_attn_rope_lut_lfm3(c.ctypes.data, s.ctypes.data, max_seq, head_dim, rope_dim,
                                        freq_base, None if rf is None else rf.ctypes.data,
                                        0 if rf is None else rf.size), "lfm_attn_rope_lut_lfm3")
    return c, s


def rope_table_lfm2(max_seq: int, head_dim: int, freq_base: float):
    c = np.empty((max_seq, head_dim // 2), np.float32)
    s = np.empty_like(c)
    check(load().lfm_attn_rope_table_lfm2(c.ctypes.data, s.ctypes.data, max_seq, head_dim, freq_base),
          "lfm_attn_rope_table_lfm2")
    return c, s


def qk_norm_rope(vec: Ptr, dst_f16: Ptr, n_heads: int, head_dim: int, norm_w: Ptr, eps: float,
                 cos_lut: Ptr, sin_lut: Ptr, pos: int, stream=None, prologue: int = PROLOGUE_FAST) -> None:
    check(load().lfm_hip_qk_norm_rope(_p(vec), _p(dst_f16), n_heads, head_dim, _p(norm_w), eps,
                                      _p(cos_lut), _p(sin_lut), pos, prologue, stream), "lfm_hip_qk_norm_rope")


def store_fp32_to_fp16(dst_f16: Ptr, src: Ptr, n: int, stream=None) -> None:
    check(load().lfm_hip_store_fp32_to_fp16(_p(dst_f16), _p(src), n, stream),
          "lfm_hip_store_fp32_to_fp16")


Q4K_BYTES, Q8K_BYTES = 144, 292  # packed block_q4_K / block_q8_K


def quantize_q8_K(x: Ptr, y_q8_K: Ptr, n_rows: int, n_cols: int, stream=None) -> None:
    """Q8_K blocks of n_rows rows of n_cols floats (n_cols % 256 == 0) into
    y_q8_K, [n_rows][n_cols / 256] packed 292-byte blocks
    (lfm2_quantize_batch_q8_K_avx2, tools/lfm2_prefill_batch.c:93-105)."""
    check(load().lfm_hip_quantize_q8_K(_p(x), _p(y_q8_K), n_rows, n_cols, stream),
          "lfm_hip_quantize_q8_K")


def matmul_q4_K(out: Ptr, w_q4_K: Ptr, n_rows: int, n_cols: int, x_q8_K: Ptr, n_tokens: int,
                stream=None) -> None:
    """out[t][r] = Q4_K row r . Q8_K token t (lfm2_matmul_1x4_prequant_mt,
    tools/lfm2_decode_1x4.c:795-813; lfm2_matmul_batch_avx2_mt,
    tools/lfm2_prefill_batch.c:598-634)."""
    check(load().lfm_hip_matmul_q4_K(_p(out), _p(w_q4_K), n_rows, n_cols, _p(x_q8_K), n_tokens,
                                     stream), "lfm_hip_matmul_q4_K")


GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_IQ4_XS = 2, 8, 12, 13, 14, 23


def matmul_prequant(out: Ptr, w: Ptr, w_type: int, n_rows: int, n_cols: int, x_q8_K: Ptr,
                    n_tokens: int, stream=None) -> None:
    """out[t][r] = row r of w (GGML type w_type) . token t of the Q8_K
    activations (lfm2_matmul_1x4_prequant_mt, tools/lfm2_decode_1x4.c:795-813)."""
    check(load().lfm_hip_matmul_prequant(_p(out), _p(w), w_type, n_rows, n_cols, _p(x_q8_K), n_tokens,
                                         stream), "lfm_hip_matmul_prequant")


def gqa_qkv_fused(outs: Sequence[Ptr], ws: Sequence[Ptr], types: Sequence[int],
                  rows: Sequence[int], n_cols: int, x_q8_K: Ptr, n_tokens: int, stream=None) -> None:
    """Q, K, V (and gate, if a fourth matrix is given) projections of the same
    Q8_K tokens in one pass (lfm2_gqa_qkv_fused_1x4_mt,
    tools/lfm2_decode_1x4.c:885-930; lfm3_gqa_qkvg_1x4_mt,
    tools/lfm3_engine.c:1545-1598).  types: GGML ids 2 (Q4_0), 8 (Q8_0),
    12 (Q4_K), 13 (Q5_K), 14 (Q6_K) or 23 (IQ4_XS)."""
    outs, ws, types, rows = list(outs), list(ws), list(types), list(rows)
    while len(outs) < 4:
        outs.append(None)
        ws.append(None)
        types.append(GGML_Q4_K)
        rows.append(0)
    t = (C.c_uint32 * 4)(*types)
    check(load().lfm_hip_gqa_qkv_fused(*[_p(o) for o in outs], *[_p(w) for w in ws], t, *rows, n_cols,
                                       _p(x_q8_K), n_tokens, stream), "lfm_hip_gqa_qkv_fused")


def qkv_prologue(q: Ptr, k: Ptr, v: Ptr, k_seq: Ptr, v_seq: Ptr, pos_0: Ptr, n_seq: int,
                 n_rows: int, n_head_q: int, n_head_kv: int, head_dim: int, q_norm_w: Ptr,
                 k_norm_w: Ptr, eps: float, cos_lut: Ptr, sin_lut: Ptr, window_len: int = 0,
                 cap: int = 0, stream=None, prologue: int = PROLOGUE_FAST) -> None:
    check(load().lfm_hip_qkv_prologue(_p(q), _p(k), _p(v), _p(k_seq), _p(v_seq), _p(pos_0), n_seq,
                                      n_rows, n_head_q, n_head_kv, head_dim, _p(q_norm_w),
                                      _p(k_norm_w), eps, _p(cos_lut), _p(sin_lut), window_len, cap,
                                      prologue, stream), "lfm_hip_qkv_prologue")


def online_gqa_f16(q: Ptr, k_cache_f16: Ptr, v_cache_f16: Ptr, xb_out: Ptr, n_head_q: int,
                   kv_mul: int, kv_dim: int, pos: int, scale: float = 0.125, stream=None) -> None:
    check(load().lfm_hip_online_gqa_f16(_p(q), _p(k_cache_f16), _p(v_cache_f16), _p(xb_out),
                                        n_head_q, kv_mul, kv_dim, pos, scale, stream),
          "lfm_hip_online_gqa_f16")


def gqa_heads(q: Ptr, k_cache: Ptr, v_cache: Ptr, k_cache_f16: Ptr, v_cache_f16: Ptr, xb: Ptr,
              n_head_q: int, kv_mul: int, head_dim: int, kv_dim: int, max_seq_len: int, pos: int,
              scale: Optional[float] = None, stream=None) -> None:
    if scale is None:
        scale = float(1.0 / np.sqrt(np.float32(head_dim)))
    check(load().lfm_hip_gqa_heads(_p(q), _p(k_cache), _p(v_cache), _p(k_cache_f16),
                                   _p(v_cache_f16), _p(xb), n_head_q, kv_mul, head_dim, kv_dim,
                                   max_seq_len, pos, scale, stream), "lfm_hip_gqa_heads")


def lfm3_online_gqa_f16_dispatch(q_batch: Ptr, gate_sig: Ptr, k_cache_f16: Ptr, v_cache_f16: Ptr,
                                 xb_out: Ptr, B: int, pos_0: int, window_len: int, swa_cap: int,
                                 n_head_q: int, n_head_kv: int, head_dim: int,
                                 stream=None) -> None:
    check(load().lfm_hip_lfm3_online_gqa_f16_dispatch(_p(q_batch), _p(gate_sig), _p(k_cache_f16),
                                                      _p(v_cache_f16), _p(xb_out), B, pos_0,
                                                      window_len, swa_cap, n_head_q, n_head_kv,
                                                      head_dim, stream),
          "lfm_hip_lfm3_online_gqa_f16_dispatch")


def gqa_f16_varlen(q: Ptr, gate: Ptr, gate_is_logit: bool, k_seq: Ptr, v_seq: Ptr, pos_0: Ptr,
                   out: Ptr, n_seq: int, n_rows: int, keys_hint: int, n_head_q: int,
                   n_head_kv: int, head_dim: int, window_len: int = 0, cap: int = 0,
                   scale: Optional[float] = None, stream=None) -> None:
    if scale is None:
        scale = float(1.0 / np.sqrt(np.float32(head_dim)))
    check(load().lfm_hip_gqa_f16_varlen(_p(q), _p(gate), int(bool(gate_is_logit)), _p(k_seq),
                                        _p(v_seq), _p(pos_0), _p(out), n_seq, n_rows,
                                        keys_hint, n_head_q, n_head_kv, head_dim, window_len,
                                        cap, scale, stream), "lfm_hip_gqa_f16_varlen")


def rope_row_gen1(head_dim: int, pos: int, theta: float):
    """Gen-1 per-call rotation row (lfm_rope_neox, src/lfm_forward.c:97-111)."""
    c = np.empty(head_dim // 2, np.float32)
    s = np.empty_like(c)
    check(load().lfm_attn_rope_row_gen1(c.ctypes.data, s.ctypes.data, head_dim, pos, theta),
          "lfm_attn_rope_row_gen1")
    return c, s


def gen1_gqa_step(q: Ptr, k: Ptr, v: Ptr, q_norm: Ptr, k_norm: Ptr, k_cache: Ptr, v_cache: Ptr,
                  attn_out: Ptr, pos: int, max_seq: int, n_heads_q: int, n_heads_kv: int, head_dim: int,
                  eps: float, cos_row: Ptr, sin_row: Ptr, stream=None) -> None:
    """Steps 2-4 of the Gen-1 lfm_gqa_step (src/lfm_forward.c:184-244) on
    device buffers: QK-RMSNorm + RoPE, FP32 KV append at pos, attention."""
    check(load().lfm_hip_gen1_gqa_step(_p(q), _p(k), _p(v), _p(q_norm), _p(k_norm), _p(k_cache), _p(v_cache),
                                       _p(attn_out), pos, max_seq, n_heads_q, n_heads_kv, head_dim, eps,
                                       _p(cos_row), _p(sin_row), stream), "lfm_hip_gen1_gqa_step")


def gqa_f16_step(q: Ptr, k: Ptr, v: Ptr, gate: Ptr, gate_is_logit: bool, k_seq: Ptr, v_seq: Ptr,
                 pos_0: Ptr, out: Ptr, n_seq: int, n_rows: int, keys_hint: int, n_head_q: int,
                 n_head_kv: int, head_dim: int, q_norm_w: Ptr, k_norm_w: Ptr, eps: float,
                 cos_lut: Ptr, sin_lut: Ptr, window_len: int = 0, cap: int = 0,
                 scale: Optional[float] = None, stream=None, prologue: int = PROLOGUE_FAST) -> None:
    """One attention step with the prologue fused: raw q/k/v rows in, the new
    rows stored in the caches, attention out (lfm_hip_gqa_f16_step)."""
    if scale is None:
        scale = float(1.0 / np.sqrt(np.float32(head_dim)))
    check(load().lfm_hip_gqa_f16_step(_p(q), _p(k), _p(v), _p(gate), int(bool(gate_is_logit)), _p(k_seq),
                                      _p(v_seq), _p(pos_0), _p(out), n_seq, n_rows, keys_hint, n_head_q,
                                      n_head_kv, head_dim, window_len, cap, scale, _p(q_norm_w),
                                      _p(k_norm_w), eps, _p(cos_lut), _p(sin_lut), prologue, stream),
          "lfm_hip_gqa_f16_step")


def gqa_f16_varlen_noalloc(q: Ptr, gate: Ptr, gate_is_logit: bool, k_seq: Ptr, v_seq: Ptr, pos_0: Ptr,
                           out: Ptr, n_seq: int, n_rows: int, keys_hint: int, n_head_q: int,
                           n_head_kv: int, head_dim: int, window_len: int = 0, cap: int = 0,
                           scale: Optional[float] = None, stream=None) -> None:
    """gqa_f16_varlen whose split partials go to the library's fixed device
    array instead of its workspace (the call allocates nothing)."""
    if scale is None:
        scale = float(1.0 / np.sqrt(np.float32(head_dim)))
    check(load().lfm_hip_gqa_f16_varlen_noalloc(_p(q), _p(gate), int(bool(gate_is_logit)), _p(k_seq),
                                                _p(v_seq), _p(pos_0), _p(out), n_seq, n_rows,
                                                keys_hint, n_head_q, n_head_kv, head_dim, window_len,
                                                cap, scale, stream), "lfm_hip_gqa_f16_varlen_noalloc")


def set_tuning(plan: Optional[str] = None, waves: int = 0, chunk: int = 0, min_tiles: int = 0,
               prefill_chain: int = 0) -> None:
    """Launch-plan overrides for tests and tuning (lfm_attn_set_tuning):
    plan None / "grid" / "balanced" / "wg", counts 0 = automatic."""
    check(load().lfm_attn_set_tuning(None if plan is None else plan.encode(), waves, chunk, min_tiles,
                                     prefill_chain), "lfm_attn_set_tuning")


class tuning:
    """Context manager: the overrides inside, automatic choice afterwards."""

    def __init__(self, plan: Optional[str] = None, waves: int = 0, chunk: int = 0, min_tiles: int = 0,
                 prefill_chain: int = 0):
        self.args = (plan, waves, chunk, min_tiles, prefill_chain)

    def __enter__(self):
        set_tuning(*self.args)
        return self

    def __exit__(self, *exc):
        set_tuning()
        return False


def plan_preview(n_seq: int, n_rows: int, n_head_q: int, n_head_kv: int, head_dim: int, window_len: int = 0,
                 keys_hint: int = 0, positions_on_device: bool = True, fused: bool = False, n_cus: int = 256):
    """(plan, waves, grid splits, grid chunk) the split-KV attention takes for
    a batch, computed on the host (lfm_attn_plan_preview)."""
    name = C.c_char_p()
    out = (C.c_uint32 * 3)()
    check(load().lfm_attn_plan_preview(n_seq, n_rows, n_head_q, n_head_kv, head_dim, window_len, keys_hint,
                                       int(positions_on_device), int(fused), n_cus, C.byref(name), out),
          "lfm_attn_plan_preview")
    return name.value.decode(), int(out[0]), int(out[1]), int(out[2])


def prefill_plan_preview(n_seq: int, n_tok: int, n_head_q: int, n_head_kv: int, head_dim: int = 128,
                         pos_0: int = 0, window_len: int = 0):
    """(query positions per tile, tiles per workgroup, short tiles dispatched
    first, workgroups) of lfm3_prefill_f16 for a prompt, computed on the host
    (lfm_attn_prefill_plan_preview)."""
    out = (C.c_uint32 * 4)()
    check(load().lfm_attn_prefill_plan_preview(n_seq, n_tok, pos_0, window_len, n_head_q, n_head_kv, head_dim, out),
          "lfm_attn_prefill_plan_preview")
    return tuple(int(x) for x in out)


def last_plan() -> str:
    """Form of this thread's last decode / step attention launch: "wg",
    "grid", "balanced" or "generic" (lfm_attn_last_plan)."""
    return load().lfm_attn_last_plan().decode()


def prefill_f16(q: Ptr, k: Ptr, v: Ptr, out: Ptr, n_seq: int, n_tok: int, pos_0: int,
                kv_seq_stride: int, n_head_q: int, n_head_kv: int, head_dim: int,
                scale: Optional[float] = None, stream=None) -> None:
    """Causal prefill: row i of each sequence (position pos_0 + i) attends
    keys [0, pos_0 + i] (tools/lfm2_prefill_batch.c:1029-1092).  q is float32
    [n_seq][n_tok][n_head_q][head_dim]; k/v are the fp16 caches."""
    if scale is None:
        scale = float(1.0 / np.sqrt(np.float32(head_dim)))
    check(load().lfm_hip_prefill_f16(_p(q), _p(k), _p(v), _p(out), n_seq, n_tok, pos_0,
                                     kv_seq_stride, n_head_q, n_head_kv, head_dim, scale, stream),
          "lfm_hip_prefill_f16")


def lfm3_prefill_f16(q: Ptr, k: Ptr, v: Ptr, gate: Optional[Ptr], gate_is_logit: bool, out: Ptr, n_seq: int,
                     n_tok: int, pos_0: int, kv_pos0: int, kv_seq_stride: int, window_len: int, n_head_q: int,
                     n_head_kv: int, head_dim: int, scale: Optional[float] = None, stream=None) -> None:
    """Causal prefill of an LFM3 layer (tools/lfm3_engine.c:1918-2055): row
    i (position p = pos_0 + i) attends keys [t_start(p), p] (the last
    window_len positions when window_len > 0), scaled by sigmoid(gate)
    (gate_is_logit) or gate.  K/V row r holds position kv_pos0 + r."""
    if scale is None:
        scale = float(1.0 / np.sqrt(np.float32(head_dim)))
    check(load().lfm_hip_lfm3_prefill_f16(_p(q), _p(k), _p(v), _p(gate), int(bool(gate_is_logit)), _p(out), n_seq,
                                          n_tok, pos_0, kv_pos0, kv_seq_stride, window_len, n_head_q, n_head_kv,
                                          head_dim, scale, stream), "lfm_hip_lfm3_prefill_f16")


def _host_ptrs(arrays) -> "C.Array":
    return (C.c_void_p * len(arrays))(*[None if a is None else int(a) for a in arrays])


def kv_cache_shift_sinks(k_caches, v_caches, n_head_kv, head_dim: int, cos_lut: Ptr, sin_lut: Ptr,
                         lut_rows: int, pos: int, n_sink: int, n_discard: int, stream=None) -> int:
    """lfm2_kv_cache_shift_sinks (tools/lfm2_runtime_features.c:744-833) on
    device caches: returns the new position.  k_caches / v_caches: per-layer
    device caches (None for a ShortConv layer); cos_lut / sin_lut: the device
    LFM2 RoPE table."""
    n = len(k_caches)
    nkv = (C.c_uint32 * n)(*n_head_kv)
    p = C.c_uint32(pos)
    check(load().lfm_hip_kv_cache_shift_sinks(_host_ptrs(k_caches), _host_ptrs(v_caches), n, nkv,
                                              head_dim, _p(cos_lut), _p(sin_lut), lut_rows,
                                              C.byref(p), n_sink, n_discard, stream),
          "lfm_hip_kv_cache_shift_sinks")
    return p.value


def lfm3_kv_cache_shift_sinks(k_caches, v_caches, n_head_kv, layer_kind, head_dim: int,
                              cos_full: Ptr, sin_full: Ptr, full_rows: int, cos_swa: Ptr,
                              sin_swa: Ptr, swa_rows: int, sliding_window: int, swa_cap: int,
                              pos: int, n_sink: int, n_discard: int, stream=None) -> int:
    """lfm3_kv_cache_shift_sinks (tools/lfm2_runtime_features.c:1055-1163) on
    device caches; layer_kind 0 = skipped, 1 = full, 2 = SWA ring.  Returns
    the new position."""
    n = len(k_caches)
    nkv = (C.c_uint32 * n)(*n_head_kv)
    kinds = (C.c_uint8 * n)(*layer_kind)
    p = C.c_uint32(pos)
    check(load().lfm_hip_lfm3_kv_cache_shift_sinks(
        _host_ptrs(k_caches), _host_ptrs(v_caches), n, nkv, kinds, head_dim, _p(cos_full),
        _p(sin_full), full_rows, _p(cos_swa), _p(sin_swa), swa_rows, sliding_window, swa_cap,
        C.byref(p), n_sink, n_discard, stream), "lfm_hip_lfm3_kv_cache_shift_sinks")
    return p.value


FNV_OFFSET_BASIS = 14695981039346656037


def fnv1a64(data: Ptr, n_bytes: int, h_in: int = FNV_OFFSET_BASIS, stream=None) -> int:
    """FNV-1a 64 of device bytes (lfm2_fnv1a_update, tools/lfm2_sys_cache.c:382-389)."""
    out = C.c_uint64(0)
    check(load().lfm_hip_fnv1a64(_p(data), n_bytes, h_in, C.byref(out), stream), "lfm_hip_fnv1a64")
    return out.value


def pointer_table(arrays: Sequence[Union["DeviceArray", int]]) -> DeviceArray:
    """Device array of device pointers (the k_seq / v_seq arguments)."""
    return DeviceArray.from_numpy(np.array([int(a) for a in arrays], dtype=np.uint64))


class CacheModel:
    """What a .lfmcache file records of the model beside the caches
    (lfm_attn_cache_model): the engine's fingerprint, its layer count (as the
    length of ctx_layer: the context layer of each attention layer, -1 for a
    ShortConv layer), n_embd, n_head_q and the ShortConv cache length."""

    def __init__(self, fingerprint, ctx_layer, n_embd, n_head_q, l_cache=3):
        self.fingerprint, self.ctx_layer = int(fingerprint), [int(x) for x in ctx_layer]
        self.n_embd, self.n_head_q, self.l_cache = n_embd, n_head_q, l_cache


class EngineContext:
    """Device-resident KV + RoPE tables for the attention layers of one model
    (lfm_attn_ctx of include/lfm_attn.h).  forward() is the per-layer
    attention step of the forward stacks with host arrays in and out."""

    def __init__(self, n_layers, n_head_q, n_head_kv, head_dim, max_seq, eps=1e-5,
                 rope_base=1e6, lfm3=False, sliding_window=0, swa_cap=0, layer_is_swa=None,
                 rope_base_swa=1e4, rope_dim=0, rope_freqs=None, prologue=PROLOGUE_FAST):
        self._keep = []
        g = Geom()
        g.n_layers, g.n_head_q, g.n_head_kv, g.head_dim = n_layers, n_head_q, n_head_kv, head_dim
        g.max_seq, g.sliding_window, g.swa_cap = max_seq, sliding_window, swa_cap
        if layer_is_swa is not None:
            arr = (C.c_uint8 * n_layers)(*[1 if x else 0 for x in layer_is_swa])
            self._keep.append(arr)
            g.layer_is_swa = C.cast(arr, C.POINTER(C.c_uint8))
        g.eps, g.rope_base, g.rope_base_swa, g.rope_dim = eps, rope_base, rope_base_swa, rope_dim
        if rope_freqs is not None:
            rf = np.ascontiguousarray(rope_freqs, np.float32)
            self._keep.append(rf)
            g.rope_freqs = rf.ctypes.data_as(C.POINTER(C.c_float))
            g.n_rope_freqs = rf.size
        g.lfm3 = 1 if lfm3 else 0
        g.prologue = int(prologue)
        self.n_head_q, self.n_head_kv, self.head_dim = n_head_q, n_head_kv, head_dim
        h = C.c_void_p()
        check(load().lfm_attn_ctx_create(C.byref(h), C.byref(g)), "lfm_attn_ctx_create")
        self.h = h.value

    def set_norms(self, layer, q_norm_w, k_norm_w):
        qn = None if q_norm_w is None else np.ascontiguousarray(q_norm_w, np.float32)
        kn = None if k_norm_w is None else np.ascontiguousarray(k_norm_w, np.float32)
        check(load().lfm_attn_ctx_set_norms(self.h, layer, None if qn is None else qn.ctypes.data,
                                            None if kn is None else kn.ctypes.data),
              "lfm_attn_ctx_set_norms")

    def forward(self, layer, pos_0, q, k, v, gate_logits=None):
        q = np.ascontiguousarray(q, np.float32)
        B = q.size // (self.n_head_q * self.head_dim)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        g = None if gate_logits is None else np.ascontiguousarray(gate_logits, np.float32)
        out = np.empty(B * self.n_head_q * self.head_dim, np.float32)
        check(load().lfm_attn_ctx_forward(self.h, layer, pos_0, B, q.ctypes.data, k.ctypes.data,
                                          v.ctypes.data, None if g is None else g.ctypes.data,
                                          out.ctypes.data), "lfm_attn_ctx_forward")
        return out

    def prefill(self, layer, pos_0, q, k, v, gate_logits=None):
        """Prompt rows pos_0 .. pos_0 + n - 1 of one layer (lfm_attn_ctx_prefill)."""
        q = np.ascontiguousarray(q, np.float32)
        n = q.size // (self.n_head_q * self.head_dim)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        g = None if gate_logits is None else np.ascontiguousarray(gate_logits, np.float32)
        out = np.empty(n * self.n_head_q * self.head_dim, np.float32)
        check(load().lfm_attn_ctx_prefill(self.h, layer, pos_0, n, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                          None if g is None else g.ctypes.data, out.ctypes.data),
              "lfm_attn_ctx_prefill")
        return out

    def kv_export(self, layer, slot, n_slots):
        row = self.n_head_kv * self.head_dim
        kh = np.empty((n_slots, row), np.uint16)
        vh = np.empty((n_slots, row), np.uint16)
        check(load().lfm_attn_ctx_kv_export(self.h, layer, slot, n_slots, kh.ctypes.data,
                                            vh.ctypes.data), "lfm_attn_ctx_kv_export")
        return kh, vh

    def kv_import(self, layer, slot, k_host, v_host):
        kh = np.ascontiguousarray(k_host, np.uint16)
        vh = np.ascontiguousarray(v_host, np.uint16)
        n = kh.size // (self.n_head_kv * self.head_dim)
        check(load().lfm_attn_ctx_kv_import(self.h, layer, slot, n, kh.ctypes.data,
                                            vh.ctypes.data), "lfm_attn_ctx_kv_import")

    def shift_sinks(self, pos, n_sink, n_discard):
        """Attention-sink eviction over every layer (src/lfm2_api.c:871-891);
        returns the new position."""
        p = C.c_uint32(pos)
        check(load().lfm_attn_ctx_shift_sinks(self.h, C.byref(p), n_sink, n_discard),
              "lfm_attn_ctx_shift_sinks")
        return p.value

    def slots(self, layer):
        """Cache slots of a layer: max_seq, or the ring size of an SWA layer."""
        n = C.c_uint32(0)
        check(load().lfm_attn_ctx_kv_device(self.h, layer, None, None, C.byref(n)),
              "lfm_attn_ctx_kv_device")
        return n.value

    # -- KV persistence --------------------------------------------------------
    @staticmethod
    def _cache_model(model):
        cm = CacheModelC()
        cm.model_fingerprint, cm.n_model_layers = model.fingerprint, len(model.ctx_layer)
        cm.n_embd, cm.n_head_q, cm.shortconv_l_cache = model.n_embd, model.n_head_q, model.l_cache
        arr = np.ascontiguousarray(model.ctx_layer, np.int32)
        cm.ctx_layer = arr.ctypes.data_as(C.POINTER(C.c_int32))
        return cm, arr

    def cache_save(self, path, model, tokens, conv_states=None, conv_ring_heads=None):
        """Write a .lfmcache v1 file of the first len(tokens) positions
        (lfm2_prompt_cache_save_ex, tools/lfm2_sys_cache.c:504-627).
        conv_states: per model layer float32 [hist, n_embd] or None."""
        cm, keep = self._cache_model(model)
        tok = np.ascontiguousarray(tokens, np.uint32)
        n = cm.n_model_layers
        conv = [None if c is None else np.ascontiguousarray(c, np.float32)
                for c in (conv_states or [None] * n)]
        cp = (C.c_void_p * n)(*[None if c is None else c.ctypes.data for c in conv])
        heads = None if conv_ring_heads is None else np.ascontiguousarray(conv_ring_heads, np.uint32)
        check(load().lfm_attn_ctx_cache_save(self.h, os.fsencode(path), C.byref(cm), tok.ctypes.data,
                                             tok.size, cp, None if heads is None else heads.ctypes.data),
              "lfm_attn_ctx_cache_save")
        del keep

    def cache_load_prefix(self, path, model, prompt, conv_states=None):
        """Restore a .lfmcache whose tokens prefix `prompt`
        (lfm2_prompt_cache_try_load_prefix_ex, tools/lfm2_sys_cache.c:650-797).
        conv_states (filled in place) as in cache_save.  Returns (matched
        position, conv ring heads); 0 when the file does not apply."""
        cm, keep = self._cache_model(model)
        pr = np.ascontiguousarray(prompt, np.uint32)
        n = cm.n_model_layers
        conv = list(conv_states) if conv_states is not None else [None] * n
        for c in conv:
            assert c is None or (c.dtype == np.float32 and c.flags.c_contiguous)
        cp = (C.c_void_p * n)(*[None if c is None else c.ctypes.data for c in conv])
        heads = np.full(n, 0xFFFFFFFF, np.uint32)
        matched = C.c_uint32(0)
        check(load().lfm_attn_ctx_cache_load_prefix(self.h, os.fsencode(path), C.byref(cm), pr.ctypes.data,
                                                    pr.size, cp, heads.ctypes.data, C.byref(matched)),
              "lfm_attn_ctx_cache_load_prefix")
        del keep
        return matched.value, heads

    def swa_slab_bytes(self):
        b = C.c_size_t(0)
        check(load().lfm_attn_ctx_swa_slab_bytes(self.h, C.byref(b)), "lfm_attn_ctx_swa_slab_bytes")
        return b.value

    def swa_slab_save(self, slab=None):
        """Checkpoint slab of the SWA rings (tools/lfm2_moe_checkpoint.c:472-506)
        into a host uint16 array (a new one when slab is None) or a DeviceArray."""
        if slab is None:
            slab = np.zeros(self.swa_slab_bytes() // 2, np.uint16)
        ptr = int(slab) if isinstance(slab, DeviceArray) else slab.ctypes.data
        check(load().lfm_attn_ctx_swa_slab_save(self.h, ptr), "lfm_attn_ctx_swa_slab_save")
        return slab

    def swa_slab_restore(self, slab):
        if isinstance(slab, DeviceArray):
            ptr = int(slab)
        else:
            slab = np.ascontiguousarray(slab, np.uint16)
            ptr = slab.ctypes.data
        check(load().lfm_attn_ctx_swa_slab_restore(self.h, ptr), "lfm_attn_ctx_swa_slab_restore")

    def close(self):
        if getattr(self, "h", None):
            load().lfm_attn_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
