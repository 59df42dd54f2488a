"""ctypes bindings for the oracle (liboracle.so) and the reference builds
(_ref/libref_attn.so, _ref/libref_gen1.so).  TEST INFRASTRUCTURE ONLY -- the
checker, never the thing measured or shipped.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref_attn.so")
REF_GEN1_SO = os.path.join(HERE, "_ref", "libref_gen1.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_u32 = C.c_uint32
_f32 = C.c_float


def build(ref: bool = True) -> None:
    """Compile the oracle (and the reference library where its sources exist)."""
    subprocess.run(["make", "-s", "-C", HERE, "oracle"] + (["ref"] if ref else []), check=True)


def _opt(arr, ptr_type):
    return None if arr is None else arr.ctypes.data_as(ptr_type)


def _cache_ptrs(caches):
    """Host pointer array over per-layer uint16 caches (None = skipped layer)."""
    for c in caches:
        assert c is None or (c.dtype == np.uint16 and c.flags.c_contiguous)
    return (C.c_void_p * len(caches))(*[None if c is None else c.ctypes.data for c in caches])


def _shift_lfm2(fn, k_caches, v_caches, n_head_kv, head_dim, cos_lut, sin_lut, pos, n_sink,
                n_discard, with_rows):
    n = len(k_caches)
    args = [_cache_ptrs(k_caches), _cache_ptrs(v_caches), n, (_u32 * n)(*n_head_kv), head_dim,
            cos_lut.ctypes.data, sin_lut.ctypes.data]
    if with_rows:
        args.append(cos_lut.shape[0])
    return fn(*args, pos, n_sink, n_discard)


def _shift_lfm3(fn, k_caches, v_caches, n_head_kv, layer_kind, head_dim, lut_full, lut_swa,
                sliding_window, swa_cap, pos, n_sink, n_discard):
    n = len(k_caches)
    (cf, sf), (cw, sw) = lut_full, lut_swa
    return fn(_cache_ptrs(k_caches), _cache_ptrs(v_caches), n, (_u32 * n)(*n_head_kv),
              (C.c_uint8 * n)(*layer_kind), head_dim, cf.ctypes.data, sf.ctypes.data, cf.shape[0],
              cw.ctypes.data, sw.ctypes.data, cw.shape[0], sliding_window, swa_cap, pos, n_sink,
              n_discard)


_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
Q4K_BYTES, Q8K_BYTES = 144, 292


def _q8k_out(n_rows, n_cols):
    return np.zeros((n_rows, (n_cols // 256) * Q8K_BYTES), np.uint8)


class Oracle:
    """Scalar C11 restatement of the reference attention path."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build(ref=False)
        L = self.lib = C.CDLL(path)
        L.orc_quantize_q8_K.argtypes = [_f32p, _u8p, _u32, _u32]
        L.orc_dot_q4_K_q8_K.restype = _f32
        L.orc_dot_q4_K_q8_K.argtypes = [_u8p, _u8p, _u32]
        L.orc_matmul_q4_K.argtypes = [_f32p, _u8p, _u32, _u32, _u8p, _u32]
        L.orc_dot_q6_K_q8_K.restype = _f32
        L.orc_dot_q6_K_q8_K.argtypes = [_u8p, _u8p, _u32]
        L.orc_matmul_q.argtypes = [_f32p, _u8p, _u32, _u32, _u32, _u8p, _u32]
        L.orc_f16_to_f32.restype = _f32
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [_f32]
        L.orc_f32_to_f16_n.argtypes = [_f32p, _u16p, C.c_size_t]
        L.orc_f16_to_f32_n.argtypes = [_u16p, _f32p, C.c_size_t]
        L.orc_rope_lut_lfm2.argtypes = [_f32p, _f32p, _u32, _u32, _f32]
        L.orc_rope_lut_lfm3.argtypes = [_f32p, _f32p, _u32, _u32, _u32, _f32, C.c_void_p, _u32]
        L.orc_qk_norm_rope.argtypes = [_f32p, C.c_void_p, _u32, _u32, C.c_void_p, _f32, _f32p, _f32p]
        L.orc_rope_table_lfm2.argtypes = [_f32p, _f32p, _u32, _u32, _f32]
        L.orc_qk_norm_rope_table.argtypes = [_f32p, C.c_void_p, _u32, _u32, C.c_void_p, _f32, _f32p,
                                             _f32p]
        L.orc_online_gqa_f16.argtypes = [_f32p, _u16p, _u16p, _f32p, _u32, _u32, _u32, _u32, _f32]
        L.orc_gqa_heads.argtypes = [_f32p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, _f32p,
                                    _u32, _u32, _u32, _u32, _u32, _f32]
        L.orc_lfm3_plan.argtypes = [_u32, _u32, _u32, _u32p]
        L.orc_lfm3_slots.restype = _u32
        L.orc_lfm3_slots.argtypes = [_u32, _u32, _u32, _u32p]
        L.orc_lfm3_online_gqa_f16.argtypes = [_f32p, C.c_void_p, _u16p, _u16p, _f32p, _u32, _u32,
                                              _u32, _u32, _u32, _u32, _u32]
        L.orc_gen1_gqa_attend.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p,
                                          _f32p, _f32p, _u32, _u32, _u32, _u32, _f32, _f32]
        L.orc_causal_rows_f16.argtypes = [_f32p, _u16p, _u16p, _f32p, _u32, _u32, _u32, _u32, _u32]
        L.orc_decode_batch_mt.argtypes = [_f32p, C.c_void_p, C.c_void_p, _u32p, _f32p, _u32, _u32,
                                          _u32, _u32, _u32]
        L.orc_kv_shift_sinks_lfm2.restype = _u32
        L.orc_kv_shift_sinks_lfm2.argtypes = [C.c_void_p, C.c_void_p, _u32, C.c_void_p, _u32,
                                              C.c_void_p, C.c_void_p, _u32, _u32, _u32]
        L.orc_kv_shift_sinks_lfm3.restype = _u32
        L.orc_kv_shift_sinks_lfm3.argtypes = [C.c_void_p, C.c_void_p, _u32, C.c_void_p, C.c_void_p,
                                              _u32, C.c_void_p, C.c_void_p, _u32, C.c_void_p,
                                              C.c_void_p, _u32, _u32, _u32, _u32, _u32, _u32]

    # -- attention-sink eviction (caches modified in place) --------------------
    def kv_shift_sinks_lfm2(self, k_caches, v_caches, n_head_kv, head_dim, lut, pos, n_sink,
                            n_discard):
        return _shift_lfm2(self.lib.orc_kv_shift_sinks_lfm2, k_caches, v_caches, n_head_kv,
                           head_dim, lut[0], lut[1], pos, n_sink, n_discard, False)

    def kv_shift_sinks_lfm3(self, k_caches, v_caches, n_head_kv, layer_kind, head_dim, lut_full,
                            lut_swa, sliding_window, swa_cap, pos, n_sink, n_discard):
        return _shift_lfm3(self.lib.orc_kv_shift_sinks_lfm3, k_caches, v_caches, n_head_kv,
                           layer_kind, head_dim, lut_full, lut_swa, sliding_window, swa_cap, pos,
                           n_sink, n_discard)

    # -- fp16 -----------------------------------------------------------------
    def f32_to_f16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=np.uint16)
        self.lib.orc_f32_to_f16_n(x.reshape(-1), out.reshape(-1), x.size)
        return out

    def f16_to_f32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, dtype=np.float32)
        self.lib.orc_f16_to_f32_n(h.reshape(-1), out.reshape(-1), h.size)
        return out

    # -- RoPE / prologue ---------------------------------------------------------
    def rope_lut_lfm2(self, max_seq, head_dim, base):
        c = np.empty((max_seq, head_dim // 2), np.float32)
        s = np.empty_like(c)
        self.lib.orc_rope_lut_lfm2(c, s, max_seq, head_dim, base)
        return c, s

    def rope_lut_lfm3(self, max_seq, head_dim, rope_dim, base, rope_freqs=None):
        c = np.empty((max_seq, head_dim // 2), np.float32)
        s = np.empty_like(c)
        rf = None if rope_freqs is None else np.ascontiguousarray(rope_freqs, np.float32)
        self.lib.orc_rope_lut_lfm3(c, s, max_seq, head_dim, rope_dim, base,
                                   _opt(rf, C.c_void_p), 0 if rf is None else rf.size)
        return c, s

    def qk_norm_rope(self, vec, n_heads, head_dim, norm_w, eps, cos_row, sin_row, store_f16=False,
                     table=False):
        """Returns the rotated fp32 heads, or the RNE fp16 store when store_f16.
        table: the production LFM2 stacks' prologue (orc_qk_norm_rope_table)."""
        v = np.ascontiguousarray(vec, np.float32).copy().reshape(-1)
        nw = None if norm_w is None else np.ascontiguousarray(norm_w, np.float32)
        dst = np.zeros(n_heads * head_dim, np.uint16) if store_f16 else None
        fn = self.lib.orc_qk_norm_rope_table if table else self.lib.orc_qk_norm_rope
        fn(v, _opt(dst, C.c_void_p), n_heads, head_dim, _opt(nw, C.c_void_p), eps,
           np.ascontiguousarray(cos_row, np.float32), np.ascontiguousarray(sin_row, np.float32))
        return dst if store_f16 else v

    def rope_table_lfm2(self, max_seq, head_dim, base):
        """Float-angle table of the production LFM2 stacks."""
        c = np.empty((max_seq, head_dim // 2), np.float32)
        s = np.empty_like(c)
        self.lib.orc_rope_table_lfm2(c, s, max_seq, head_dim, base)
        return c, s

    # -- attention ---------------------------------------------------------------
    def online_gqa_f16(self, q, k16, v16, n_head_q, kv_mul, kv_dim, pos, scale=0.125):
        out = np.zeros(n_head_q * 64, np.float32)
        self.lib.orc_online_gqa_f16(np.ascontiguousarray(q, np.float32).reshape(-1),
                                    k16.reshape(-1), v16.reshape(-1), out, n_head_q, kv_mul,
                                    kv_dim, pos, scale)
        return out

    def gqa_heads(self, q, n_head_q, kv_mul, head_dim, kv_dim, pos, k32=None, v32=None,
                  k16=None, v16=None, out=None):
        o = np.zeros(n_head_q * head_dim, np.float32) if out is None else out.copy()
        arrs = [None if a is None else np.ascontiguousarray(a).reshape(-1)
                for a in (k32, v32, k16, v16)]
        self.lib.orc_gqa_heads(np.ascontiguousarray(q, np.float32).reshape(-1),
                               *[_opt(a, C.c_void_p) for a in arrs], o, n_head_q, kv_mul,
                               head_dim, kv_dim, pos, 1.0 / np.sqrt(np.float32(head_dim)))
        return o

    def lfm3_plan(self, abs_pos, window, cap):
        out = np.zeros(5, np.uint32)
        self.lib.orc_lfm3_plan(abs_pos, window, cap, out)
        return tuple(int(x) for x in out)

    def lfm3_slots(self, abs_pos, window, cap):
        buf = np.zeros(abs_pos + 1, np.uint32)
        n = self.lib.orc_lfm3_slots(abs_pos, window, cap, buf)
        return buf[:n]

    def lfm3_online_gqa_f16(self, q, gate, k16, v16, B, pos_0, window, cap, n_head_q, n_head_kv,
                            head_dim):
        out = np.zeros(B * n_head_q * head_dim, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32).reshape(-1)
        self.lib.orc_lfm3_online_gqa_f16(np.ascontiguousarray(q, np.float32).reshape(-1),
                                         _opt(g, C.c_void_p), k16.reshape(-1), v16.reshape(-1),
                                         out, B, pos_0, window, cap, n_head_q, n_head_kv,
                                         head_dim)
        return out

    def gen1_gqa_attend(self, q, k, v, q_norm, k_norm, k_cache, v_cache, pos, nq, nkv, hd, eps,
                        theta):
        out = np.zeros(nq * hd, np.float32)
        q = np.ascontiguousarray(q, np.float32).copy()
        k = np.ascontiguousarray(k, np.float32).copy()
        qn = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
        kn = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
        self.lib.orc_gen1_gqa_attend(out, q, k, np.ascontiguousarray(v, np.float32),
                                     _opt(qn, C.c_void_p), _opt(kn, C.c_void_p),
                                     k_cache.reshape(-1), v_cache.reshape(-1), pos, nq, nkv, hd,
                                     eps, theta)
        return out

    def causal_rows_f16(self, q_rows, k16, v16, n_rows, pos_0, n_head_q, n_head_kv, head_dim):
        out = np.zeros(n_rows * n_head_q * head_dim, np.float32)
        self.lib.orc_causal_rows_f16(np.ascontiguousarray(q_rows, np.float32).reshape(-1),
                                     k16.reshape(-1), v16.reshape(-1), out, n_rows, pos_0,
                                     n_head_q, n_head_kv, head_dim)
        return out

    def decode_batch_mt(self, q, k_list, v_list, pos, n_head_q, n_head_kv, head_dim, n_threads):
        n_seq = len(k_list)
        kp = (C.c_void_p * n_seq)(*[k.ctypes.data for k in k_list])
        vp = (C.c_void_p * n_seq)(*[v.ctypes.data for v in v_list])
        out = np.zeros(n_seq * n_head_q * head_dim, np.float32)
        self.lib.orc_decode_batch_mt(np.ascontiguousarray(q, np.float32).reshape(-1), kp, vp,
                                     np.ascontiguousarray(pos, np.uint32), out, n_seq, n_head_q,
                                     n_head_kv, head_dim, n_threads)
        return out


def _quantize_q8_K(self, x):
    """x: float32 [n_rows, n_cols] -> uint8 [n_rows, n_cols/256 * 292] (packed blocks)."""
    x = np.ascontiguousarray(x, np.float32)
    y = _q8k_out(*x.shape)
    self._quant(x, y, x.shape[0], x.shape[1])
    return y


def _orc_quant(self, x, y, n_rows, n_cols):
    self.lib.orc_quantize_q8_K(x, y, n_rows, n_cols)


Oracle._quant = _orc_quant
Oracle.quantize_q8_K = _quantize_q8_K


def _orc_dot(self, w_row, x_q8, n_cols):
    return float(self.lib.orc_dot_q4_K_q8_K(np.ascontiguousarray(w_row, np.uint8),
                                             np.ascontiguousarray(x_q8, np.uint8), n_cols))


def _orc_matmul(self, w, x_q8, n_cols):
    """w: uint8 [n_rows, nb*144]; x_q8: uint8 [B, nb*292] -> float32 [B, n_rows]."""
    w = np.ascontiguousarray(w, np.uint8)
    x_q8 = np.ascontiguousarray(x_q8, np.uint8)
    out = np.zeros((x_q8.shape[0], w.shape[0]), np.float32)
    self.lib.orc_matmul_q4_K(out, w, w.shape[0], n_cols, x_q8, x_q8.shape[0])
    return out


def _orc_dot6(self, w_row, x_q8, n_cols):
    return float(self.lib.orc_dot_q6_K_q8_K(np.ascontiguousarray(w_row, np.uint8),
                                             np.ascontiguousarray(x_q8, np.uint8), n_cols))


def _orc_matmul_q(self, w, qtype, x_q8, n_cols):
    """GGML type 2, 8, 12, 13, 14 or 23 rows: w uint8 [n_rows, row bytes] -> float32 [B, n_rows]."""
    w = np.ascontiguousarray(w, np.uint8)
    x_q8 = np.ascontiguousarray(x_q8, np.uint8)
    out = np.zeros((x_q8.shape[0], w.shape[0]), np.float32)
    self.lib.orc_matmul_q(out, w, qtype, w.shape[0], n_cols, x_q8, x_q8.shape[0])
    return out


Oracle.dot_q4_K = _orc_dot
Oracle.matmul_q4_K = _orc_matmul
Oracle.dot_q6_K = _orc_dot6
Oracle.matmul_q = _orc_matmul_q


class RefGen1:
    """The reference's Gen-1 FP32 step (src/lfm_forward.c, ref_gen1_shim.c)."""

    @staticmethod
    def available(path: str = REF_GEN1_SO) -> bool:
        return os.path.exists(path)

    def __init__(self, path: str = REF_GEN1_SO):
        L = self.lib = C.CDLL(path)
        L.ref_gen1_rope_neox.argtypes = [_f32p, _u32, _u32, _f32]
        L.ref_gen1_rmsnorm.argtypes = [_f32p, _f32p, C.c_void_p, _u32, _f32]
        L.ref_gen1_gqa_step.restype = C.c_int
        L.ref_gen1_gqa_step.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p,
                                        _f32p, _f32p, _u32, _u32, _u32, _u32, _u32, _u32, _f32, _f32]

    def rope_row(self, head_dim, pos, theta):
        """cos, sin of lfm_rope_neox's angles: the rotation of (1, 0) pairs."""
        v = np.zeros(head_dim, np.float32)
        v[:head_dim // 2] = 1.0
        self.lib.ref_gen1_rope_neox(v, head_dim, pos, theta)
        return v[:head_dim // 2].copy(), v[head_dim // 2:].copy()

    def rmsnorm(self, x, weight, eps):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        w = None if weight is None else np.ascontiguousarray(weight, np.float32)
        self.lib.ref_gen1_rmsnorm(out, x, _opt(w, C.c_void_p), x.size, eps)
        return out

    def gqa_step(self, x_norm, wq, wk, wv, wo, q_norm, k_norm, k_cache, v_cache, pos, nq, nkv, hd, eps, theta):
        """lfm_gqa_step with F32 weights; k_cache/v_cache are updated in place."""
        D = x_norm.size
        out = np.zeros(D, np.float32)
        qn = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
        kn = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
        rc = self.lib.ref_gen1_gqa_step(out, np.ascontiguousarray(x_norm, np.float32),
                                        *[np.ascontiguousarray(w, np.float32).reshape(-1) for w in (wq, wk, wv, wo)],
                                        _opt(qn, C.c_void_p), _opt(kn, C.c_void_p), k_cache.reshape(-1),
                                        v_cache.reshape(-1), pos, k_cache.shape[0], D, nq, nkv, hd, eps, theta)
        assert rc == 0
        return out


class Reference:
    """The reference's own kernels, compiled from /root/reference (ref_shim.c)."""

    @staticmethod
    def available(path: str = REF_SO) -> bool:
        return os.path.exists(path)

    def __init__(self, path: str = REF_SO):
        L = self.lib = C.CDLL(path)
        L.ref_has_avx2.restype = C.c_int
        L.ref_rope_lut_lfm2.argtypes = [_f32p, _f32p, _u32, _u32, _f32]
        L.ref_rope_lut_lfm3.argtypes = [_f32p, _f32p, _u32, _u32, _u32, _f32, C.c_void_p, _u32]
        L.ref_qk_norm_rope_lfm2.argtypes = [_f32p, C.c_void_p, _u32, C.c_void_p, _f32, _f32p,
                                            _f32p, _u32, _u32, C.c_int]
        L.ref_qk_norm_rope_lfm3.argtypes = [_f32p, C.c_void_p, _u32, _u32, C.c_void_p, _f32, _f32p,
                                            _f32p, _u32, _u32, C.c_int]
        L.ref_store_fp32_to_fp16.argtypes = [_u16p, _f32p, _u32]
        L.ref_time_attn.argtypes = [C.c_int, C.c_int, _f32p, C.c_void_p, C.c_void_p, C.c_void_p, _u32p, _f32p,
                                    _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                    C.POINTER(C.c_double), C.POINTER(_u32)]
        L.ref_rope_table_lfm2.argtypes = [_f32p, _f32p, _u32, _u32, _u32, _f32, C.c_int]
        L.ref_qk_norm_rope_table.argtypes = [_f32p, _u32, _u32, C.c_void_p, _f32, _f32p, _f32p, _u32,
                                             C.c_int]
        L.ref_fp16_to_fp32.restype = _f32
        L.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        L.ref_online_gqa_f16.argtypes = [_f32p, _u16p, _u16p, _f32p, _u32, _u32, _u32, _u32, _u32]
        L.ref_gqa_heads.argtypes = [_f32p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, _f32p,
                                    _u32, _u32, _u32, _u32, _u32, _u32, _u32]
        L.ref_lfm3_dispatch.argtypes = [_f32p, C.c_void_p, _u16p, _u16p, _f32p, _u32, _u32, _u32,
                                        _u32, _u32, _u32, _u32, _u32]
        L.ref_time_decode_batch.restype = C.c_double
        L.ref_time_decode_batch.argtypes = [_f32p, C.c_void_p, C.c_void_p, _u32p, _f32p, _u32,
                                            _u32, _u32, _u32, _u32, C.POINTER(_u32)]
        L.ref_time_decode_batch_fair.restype = C.c_double
        L.ref_time_decode_batch_fair.argtypes = [_f32p, C.c_void_p, C.c_void_p, _u32p, _f32p, _u32,
                                                 _u32, _u32, _u32, _u32]
        L.ref_kv_shift_sinks_lfm2.restype = _u32
        L.ref_kv_shift_sinks_lfm2.argtypes = [C.c_void_p, C.c_void_p, _u32, C.c_void_p, _u32,
                                              C.c_void_p, C.c_void_p, _u32, _u32, _u32, _u32]
        L.ref_kv_shift_sinks_lfm3.restype = _u32
        L.ref_kv_shift_sinks_lfm3.argtypes = [C.c_void_p, C.c_void_p, _u32, C.c_void_p, C.c_void_p,
                                              _u32, C.c_void_p, C.c_void_p, _u32, C.c_void_p,
                                              C.c_void_p, _u32, _u32, _u32, _u32, _u32, _u32]
        L.ref_quantize_q8_K.argtypes = [_f32p, _u8p, _u32, _u32]
        L.ref_dot_q4_K_avx2.restype = _f32
        L.ref_dot_q4_K_avx2.argtypes = [_u8p, _u8p, _u32]
        L.ref_matmul_q4_K_prequant.argtypes = [_f32p, _u8p, _u32, _u32, _u8p]
        L.ref_matmul_q4_K_batch.argtypes = [_f32p, _u8p, _u32, _u32, _f32p, _u32]
        L.ref_dot_q6_K_avx2.restype = _f32
        L.ref_dot_q6_K_avx2.argtypes = [_u8p, _u8p, _u32]
        self.has_avx2 = bool(L.ref_has_avx2())

    def kv_shift_sinks_lfm2(self, k_caches, v_caches, n_head_kv, head_dim, lut, pos, n_sink,
                            n_discard):
        return _shift_lfm2(self.lib.ref_kv_shift_sinks_lfm2, k_caches, v_caches, n_head_kv,
                           head_dim, lut[0], lut[1], pos, n_sink, n_discard, True)

    def kv_shift_sinks_lfm3(self, k_caches, v_caches, n_head_kv, layer_kind, head_dim, lut_full,
                            lut_swa, sliding_window, swa_cap, pos, n_sink, n_discard):
        return _shift_lfm3(self.lib.ref_kv_shift_sinks_lfm3, k_caches, v_caches, n_head_kv,
                           layer_kind, head_dim, lut_full, lut_swa, sliding_window, swa_cap, pos,
                           n_sink, n_discard)

    def rope_lut_lfm2(self, max_seq, head_dim, base):
        c = np.empty((max_seq, head_dim // 2), np.float32)
        s = np.empty_like(c)
        assert self.lib.ref_rope_lut_lfm2(c, s, max_seq, head_dim, base) == 0
        return c, s

    def rope_lut_lfm3(self, max_seq, head_dim, rope_dim, base, rope_freqs=None):
        c = np.empty((max_seq, head_dim // 2), np.float32)
        s = np.empty_like(c)
        rf = None if rope_freqs is None else np.ascontiguousarray(rope_freqs, np.float32)
        assert self.lib.ref_rope_lut_lfm3(c, s, max_seq, head_dim, rope_dim, base,
                                          _opt(rf, C.c_void_p),
                                          0 if rf is None else rf.size) == 0
        return c, s

    def qk_norm_rope(self, vec, n_heads, head_dim, norm_w, eps, cos_lut, sin_lut, pos,
                     store_f16=False, scalar=False):
        v = np.ascontiguousarray(vec, np.float32).copy().reshape(-1)
        nw = None if norm_w is None else np.ascontiguousarray(norm_w, np.float32)
        dst = np.zeros(n_heads * head_dim, np.uint16) if store_f16 else None
        c = np.ascontiguousarray(cos_lut, np.float32)
        s = np.ascontiguousarray(sin_lut, np.float32)
        if head_dim == 64 and c.shape[1] == 32 and not getattr(self, "_force_lfm3", False):
            rc = self.lib.ref_qk_norm_rope_lfm2(v, _opt(dst, C.c_void_p), n_heads,
                                                _opt(nw, C.c_void_p), eps, c, s, c.shape[0], pos,
                                                int(scalar))
        else:
            rc = self.lib.ref_qk_norm_rope_lfm3(v, _opt(dst, C.c_void_p), n_heads, head_dim,
                                                _opt(nw, C.c_void_p), eps, c, s, c.shape[0], pos,
                                                int(scalar))
        assert rc == 0
        return dst if store_f16 else v

    def store_f16(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty(x.size, np.uint16)
        self.lib.ref_store_fp32_to_fp16(out, x, x.size)
        return out

    KIND = {"lfm2_decode": 0, "lfm2_rows": 1, "lfm3_decode": 2}

    def time_attn(self, kind, fair, q, k_list, v_list, pos0, n_head_q, n_head_kv, head_dim, n_rows=1,
                  gate=None, window=0, cap=0, n_threads=1, warm=3, reps=10):
        """The reference's CPU attention over a multi-sequence batch
        (ref_time_attn): kind "lfm2_decode" / "lfm2_rows" / "lfm3_decode";
        fair False = the engine's dispatch per sequence (per row), True = every
        item on all threads.  Returns (per-pass seconds [reps], threads, out)."""
        n_seq = len(k_list)
        q = np.ascontiguousarray(q, np.float32).reshape(-1)
        out = np.zeros(n_seq * n_rows * n_head_q * head_dim, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32).reshape(-1)
        kp = (C.c_void_p * n_seq)(*[k.ctypes.data for k in k_list])
        vp = (C.c_void_p * n_seq)(*[v.ctypes.data for v in v_list])
        max_seq = max(int(k.size) // (n_head_kv * head_dim) for k in k_list)
        times = (C.c_double * reps)()
        used = _u32(0)
        rc = self.lib.ref_time_attn(self.KIND[kind], int(fair), q, _opt(g, C.c_void_p), kp, vp,
                                    np.ascontiguousarray(pos0, np.uint32), out, n_seq, n_rows, n_head_q, n_head_kv,
                                    head_dim, window, cap, max_seq, n_threads, warm, reps, times, C.byref(used))
        assert rc == 0
        return np.array(times[:], np.float64), int(used.value), out

    def rope_table_lfm2(self, max_seq, head_dim, base, which=0, n_head_q=4):
        """which 0: lfm2_batch_state_init's table, 1: lfm2_state_init's."""
        c = np.empty((max_seq, head_dim // 2), np.float32)
        s = np.empty_like(c)
        assert self.lib.ref_rope_table_lfm2(c, s, max_seq, n_head_q, head_dim, base, which) == 0
        return c, s

    def qk_norm_rope_table(self, vec, n_heads, head_dim, norm_w, eps, cos_tab, sin_tab, pos, which=0):
        """which 0: lfm2_qk_norm_and_rope_table, 1: lfm2_qk_norm_and_rope (in place on a copy)."""
        v = np.ascontiguousarray(vec, np.float32).copy().reshape(-1)
        nw = None if norm_w is None else np.ascontiguousarray(norm_w, np.float32)
        assert self.lib.ref_qk_norm_rope_table(v, n_heads, head_dim, _opt(nw, C.c_void_p), eps,
                                               np.ascontiguousarray(cos_tab, np.float32),
                                               np.ascontiguousarray(sin_tab, np.float32), pos, which) == 0
        return v

    def online_gqa_f16(self, q, k16, v16, n_head_q, kv_mul, kv_dim, pos, n_threads=2):
        out = np.zeros(n_head_q * 64, np.float32)
        self.lib.ref_online_gqa_f16(np.ascontiguousarray(q, np.float32).reshape(-1),
                                    k16.reshape(-1), v16.reshape(-1), out, n_head_q, kv_mul,
                                    kv_dim, pos, n_threads)
        return out

    def gqa_heads(self, q, n_head_q, kv_mul, head_dim, kv_dim, max_seq, pos, k32=None, v32=None,
                  k16=None, v16=None, n_threads=2):
        out = np.zeros(n_head_q * head_dim, np.float32)
        arrs = [None if a is None else np.ascontiguousarray(a).reshape(-1)
                for a in (k32, v32, k16, v16)]
        self.lib.ref_gqa_heads(np.ascontiguousarray(q, np.float32).reshape(-1),
                               *[_opt(a, C.c_void_p) for a in arrs], out, n_head_q, kv_mul,
                               head_dim, kv_dim, max_seq, pos, n_threads)
        return out

    def lfm3_dispatch(self, q, gate, k16, v16, B, pos_0, window, cap, n_head_q, n_head_kv,
                      head_dim, n_threads=2):
        out = np.zeros(B * n_head_q * head_dim, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32).reshape(-1)
        self.lib.ref_lfm3_dispatch(np.ascontiguousarray(q, np.float32).reshape(-1),
                                   _opt(g, C.c_void_p), k16.reshape(-1), v16.reshape(-1), out, B,
                                   pos_0, window, cap, n_head_q, n_head_kv, head_dim, n_threads)
        return out

    def time_decode_batch(self, q, k_list, v_list, pos, n_head_q, n_head_kv, n_threads, reps):
        n_seq = len(k_list)
        kp = (C.c_void_p * n_seq)(*[k.ctypes.data for k in k_list])
        vp = (C.c_void_p * n_seq)(*[v.ctypes.data for v in v_list])
        out = np.zeros(n_seq * n_head_q * 64, np.float32)
        used = _u32(0)
        dt = self.lib.ref_time_decode_batch(np.ascontiguousarray(q, np.float32).reshape(-1), kp,
                                            vp, np.ascontiguousarray(pos, np.uint32), out, n_seq,
                                            n_head_q, n_head_kv, n_threads, reps, C.byref(used))
        return dt, int(used.value), out

    def time_decode_batch_fair(self, q, k_list, v_list, pos, n_head_q, n_head_kv, n_threads, reps):
        """The reference's decode worker over every (sequence, 4-head group)
        item of the batch across n_threads threads; fastest of reps passes."""
        n_seq = len(k_list)
        kp = (C.c_void_p * n_seq)(*[k.ctypes.data for k in k_list])
        vp = (C.c_void_p * n_seq)(*[v.ctypes.data for v in v_list])
        out = np.zeros(n_seq * n_head_q * 64, np.float32)
        dt = self.lib.ref_time_decode_batch_fair(np.ascontiguousarray(q, np.float32).reshape(-1), kp,
                                                 vp, np.ascontiguousarray(pos, np.uint32), out, n_seq,
                                                 n_head_q, n_head_kv, n_threads, reps)
        return dt, out


def _ref_quant(self, x, y, n_rows, n_cols):
    self.lib.ref_quantize_q8_K(x, y, n_rows, n_cols)


def _ref_dot(self, w_row, x_q8, n_cols):
    return float(self.lib.ref_dot_q4_K_avx2(np.ascontiguousarray(w_row, np.uint8),
                                             np.ascontiguousarray(x_q8, np.uint8), n_cols))


def _ref_matmul_prequant(self, w, x_q8, n_cols):
    """The engine's decode projection (1x4 rows): x_q8 uint8 [1, nb*292] -> float32 [1, n_rows]."""
    w = np.ascontiguousarray(w, np.uint8)
    out = np.zeros((1, w.shape[0]), np.float32)
    self.lib.ref_matmul_q4_K_prequant(out, w, w.shape[0], n_cols, np.ascontiguousarray(x_q8, np.uint8))
    return out


def _ref_matmul_batch(self, w, x):
    """The engine's batched projection from fp32 tokens x [B <= 8, n_cols] -> [B, n_rows]."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    assert x.shape[0] <= 8
    out = np.zeros((x.shape[0], w.shape[0]), np.float32)
    self.lib.ref_matmul_q4_K_batch(out, w, w.shape[0], x.shape[1], x, x.shape[0])
    return out


Reference._quant = _ref_quant
Reference.quantize_q8_K = _quantize_q8_K
Reference.dot_q4_K = _ref_dot
Reference.matmul_q4_K_prequant = _ref_matmul_prequant
Reference.matmul_q4_K_batch = _ref_matmul_batch


def _ref_dot6(self, w_row, x_q8, n_cols):
    return float(self.lib.ref_dot_q6_K_avx2(np.ascontiguousarray(w_row, np.uint8),
                                             np.ascontiguousarray(x_q8, np.uint8), n_cols))


Reference.dot_q6_K = _ref_dot6


# -- KV persistence: .lfmcache v1 prompt cache and the checkpoint SWA slab ----------
class CacheModel:
    """The model fields the .lfmcache format and the fingerprint read
    (LFM2Config of the reference): layer_kind 0 ShortConv, 1 full attention,
    2 sliding-window attention; n_head_kv per layer (0 for ShortConv)."""

    def __init__(self, layer_kind, n_head_kv, head_dim, n_embd, n_head_q, l_cache=3,
                 sliding_window=0, is_lfm3=False, n_vocab=65536):
        self.layer_kind = np.ascontiguousarray(layer_kind, np.uint8)
        self.n_head_kv = np.ascontiguousarray(n_head_kv, np.uint32)
        self.n_layers = int(self.layer_kind.size)
        self.head_dim, self.n_embd, self.n_head_q = head_dim, n_embd, n_head_q
        self.l_cache, self.sliding_window, self.is_lfm3 = l_cache, sliding_window, bool(is_lfm3)
        self.n_vocab = n_vocab

    @property
    def hist_len(self):
        return self.l_cache - 1 if self.l_cache > 1 else 2

    def args(self):
        return (self.n_layers, self.n_head_kv, self.layer_kind, self.head_dim, self.n_embd,
                self.n_head_q, self.l_cache, self.sliding_window)


def _f32_ptrs(arrs):
    for a in arrs:
        assert a is None or (a.dtype == np.float32 and a.flags.c_contiguous)
    return (C.c_void_p * len(arrs))(*[None if a is None else a.ctypes.data for a in arrs])


def _heads_arr(heads, n):
    return None if heads is None else np.ascontiguousarray(heads, np.uint32)


_CACHE_GEOM = [_u32, _u32p, _u8p, _u32, _u32, _u32, _u32, _u32]


def _bind_cache(L, prefix, fp_arg):
    fp = [C.c_uint64] if fp_arg else []
    save = getattr(L, prefix + "prompt_cache_save")
    save.restype = C.c_int
    load = getattr(L, prefix + "prompt_cache_load")
    load.restype = _u32
    if fp_arg:  # oracle: (path, fingerprint, geometry...)
        save.argtypes = [C.c_char_p] + fp + _CACHE_GEOM + [_u32p, _u32, C.c_void_p, C.c_void_p,
                                                           C.c_void_p, C.c_void_p, _u32]
        load.argtypes = [C.c_char_p] + fp + _CACHE_GEOM + [_u32p, _u32, _u32, C.c_void_p, C.c_void_p,
                                                           C.c_void_p, C.c_void_p, _u32]
    else:  # reference: (path, geometry..., is_lfm3, ...)
        save.argtypes = [C.c_char_p] + _CACHE_GEOM + [C.c_int, _u32p, _u32, C.c_void_p, C.c_void_p,
                                                      C.c_void_p, C.c_void_p, _u32]
        load.argtypes = [C.c_char_p] + _CACHE_GEOM + [C.c_int, _u32p, _u32, _u32, C.c_void_p,
                                                      C.c_void_p, C.c_void_p, C.c_void_p, _u32]


def _pc_save(self, path, model, tokens, conv, k, v, conv_heads=None, swa_cap=0, fingerprint=None):
    """Write a prompt cache; conv/k/v are per-layer lists (None where a layer has none)."""
    tokens = np.ascontiguousarray(tokens, np.uint32)
    n = model.n_layers
    conv = list(conv) + [None] * (n - len(conv))
    heads = _heads_arr(conv_heads, n)
    hp = None if heads is None else heads.ctypes.data
    if isinstance(self, Oracle):
        fp = self.model_fingerprint(model) if fingerprint is None else fingerprint
        ok = self.lib.orc_prompt_cache_save(path.encode(), fp, *model.args(), tokens, tokens.size,
                                            _f32_ptrs(conv), hp, _cache_ptrs(k), _cache_ptrs(v), swa_cap)
    else:
        ok = self.lib.ref_prompt_cache_save(path.encode(), *model.args(), int(model.is_lfm3), tokens,
                                            tokens.size, _f32_ptrs(conv), hp, _cache_ptrs(k),
                                            _cache_ptrs(v), swa_cap)
    return bool(ok)


def _pc_load(self, path, model, prompt, max_seq, conv, k, v, swa_cap=0, fingerprint=None):
    """Load into the given buffers (modified in place); returns (matched, conv_heads)."""
    prompt = np.ascontiguousarray(prompt, np.uint32)
    n = model.n_layers
    conv = list(conv) + [None] * (n - len(conv))
    heads = np.full(n, 0xFFFFFFFF, np.uint32)
    if isinstance(self, Oracle):
        fp = self.model_fingerprint(model) if fingerprint is None else fingerprint
        m = self.lib.orc_prompt_cache_load(path.encode(), fp, *model.args(), prompt, prompt.size,
                                           max_seq, _f32_ptrs(conv), heads.ctypes.data,
                                           _cache_ptrs(k), _cache_ptrs(v), swa_cap)
    else:
        m = self.lib.ref_prompt_cache_load(path.encode(), *model.args(), int(model.is_lfm3), prompt,
                                           prompt.size, max_seq, _f32_ptrs(conv), heads.ctypes.data,
                                           _cache_ptrs(k), _cache_ptrs(v), swa_cap)
    return int(m), heads


def _orc_fingerprint(self, model, arch=None):
    arch = arch or ("lfm3" if model.is_lfm3 else "lfm2")
    is_swa = np.ascontiguousarray(model.layer_kind == 2, np.uint8)
    return int(self.lib.orc_model_fingerprint(arch.encode(), model.n_layers, model.n_embd, model.n_vocab,
                                              model.n_head_q, model.l_cache, model.n_head_kv,
                                              int(model.is_lfm3), model.head_dim,
                                              model.sliding_window, is_swa))


def _ref_fingerprint(self, model):
    return int(self.lib.ref_model_fingerprint(model.n_layers, model.n_head_kv, model.layer_kind,
                                              model.head_dim, model.n_embd, model.n_head_q,
                                              model.l_cache, model.sliding_window,
                                              int(model.is_lfm3)))


def _orc_fnv1a(self, data, h=14695981039346656037):
    b = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else data
    b = np.ascontiguousarray(b).view(np.uint8)
    return int(self.lib.orc_fnv1a(h, b.ctypes.data, b.size))


def _orc_slab(self, model, swa_cap, k, v, slab=None):
    """Checkpoint SWA slab of the caches (slab=None: a new one), or restore
    the caches from `slab` when it is given."""
    n = self.lib.orc_checkpoint_swa_slab(None, model.n_layers, model.n_head_kv, model.layer_kind,
                                         model.head_dim, swa_cap, _cache_ptrs(k), _cache_ptrs(v), 0)
    restore = slab is not None
    out = np.ascontiguousarray(slab, np.uint16) if restore else np.zeros(n, np.uint16)
    assert out.size == n
    self.lib.orc_checkpoint_swa_slab(out.ctypes.data, model.n_layers, model.n_head_kv,
                                     model.layer_kind, model.head_dim, swa_cap, _cache_ptrs(k),
                                     _cache_ptrs(v), int(restore))
    return out


def _ref_slab_save(self, model, k, v):
    n = self.lib.ref_checkpoint_swa_save(None, *model.args(), _cache_ptrs(k), _cache_ptrs(v))
    out = np.zeros(n, np.uint16)
    self.lib.ref_checkpoint_swa_save(out.ctypes.data, *model.args(), _cache_ptrs(k), _cache_ptrs(v))
    return out


def _ref_slab_restore(self, model, slab, k, v):
    slab = np.ascontiguousarray(slab, np.uint16)
    return bool(self.lib.ref_checkpoint_swa_restore(slab.ctypes.data, *model.args(), _cache_ptrs(k),
                                                    _cache_ptrs(v)))


def _orc_cache_init(self):
    L = self.lib
    _bind_cache(L, "orc_", True)
    L.orc_fnv1a.restype = C.c_uint64
    L.orc_fnv1a.argtypes = [C.c_uint64, C.c_void_p, C.c_size_t]
    L.orc_model_fingerprint.restype = C.c_uint64
    L.orc_model_fingerprint.argtypes = [C.c_char_p, _u32, _u32, _u32, _u32, _u32, _u32p, C.c_int, _u32,
                                        _u32, _u8p]
    L.orc_checkpoint_swa_slab.restype = C.c_size_t
    L.orc_checkpoint_swa_slab.argtypes = [C.c_void_p, _u32, _u32p, _u8p, _u32, _u32, C.c_void_p,
                                          C.c_void_p, C.c_int]


def _ref_cache_init(self):
    L = self.lib
    _bind_cache(L, "ref_", False)
    L.ref_model_fingerprint.restype = C.c_uint64
    L.ref_model_fingerprint.argtypes = _CACHE_GEOM + [C.c_int]
    L.ref_checkpoint_swa_save.restype = C.c_size_t
    L.ref_checkpoint_swa_save.argtypes = [C.c_void_p] + _CACHE_GEOM + [C.c_void_p, C.c_void_p]
    L.ref_checkpoint_swa_restore.restype = C.c_int
    L.ref_checkpoint_swa_restore.argtypes = [C.c_void_p] + _CACHE_GEOM + [C.c_void_p, C.c_void_p]


def _wrap_init(cls, extra):
    base = cls.__init__

    def __init__(self, *a, **kw):
        base(self, *a, **kw)
        extra(self)

    cls.__init__ = __init__


_wrap_init(Oracle, _orc_cache_init)
_wrap_init(Reference, _ref_cache_init)
Oracle.prompt_cache_save = Reference.prompt_cache_save = _pc_save
Oracle.prompt_cache_load = Reference.prompt_cache_load = _pc_load
Oracle.model_fingerprint = _orc_fingerprint
Oracle.fnv1a = _orc_fnv1a
Oracle.checkpoint_swa_slab = _orc_slab
Reference.model_fingerprint = _ref_fingerprint
Reference.checkpoint_swa_save = _ref_slab_save
Reference.checkpoint_swa_restore = _ref_slab_restore


# -- other weight types of the projections (GGML ids 2, 8, 13, 23) ---------------
Q_BLOCK_BYTES = {2: 144, 8: 272, 12: 144, 13: 176, 14: 210, 23: 136}  # bytes per 256 weights


def _orc_types_init(self):
    L = self.lib
    for n in ("q4_0", "q8_0", "q5_K", "iq4_xs"):
        f = getattr(L, f"orc_dot_{n}_q8_K")
        f.restype = _f32
        f.argtypes = [_u8p, _u8p, _u32]


def _ref_types_init(self):
    L = self.lib
    for n in ("q4_0", "q8_0", "q5_K", "iq4_xs"):
        f = getattr(L, f"ref_dot_{n}_avx2")
        f.restype = _f32
        f.argtypes = [_u8p, _u8p, _u32]
    L.ref_matmul_prequant_type.argtypes = [_f32p, _u8p, _u32, _u32, _u32, _u8p]


_DOT_NAMES = {2: "q4_0", 8: "q8_0", 13: "q5_K", 23: "iq4_xs"}


def _orc_dot_type(self, w_row, qtype, x_q8, n_cols):
    f = getattr(self.lib, f"orc_dot_{_DOT_NAMES[qtype]}_q8_K")
    return float(f(np.ascontiguousarray(w_row, np.uint8), np.ascontiguousarray(x_q8, np.uint8), n_cols))


def _ref_dot_type(self, w_row, qtype, x_q8, n_cols):
    f = getattr(self.lib, f"ref_dot_{_DOT_NAMES[qtype]}_avx2")
    return float(f(np.ascontiguousarray(w_row, np.uint8), np.ascontiguousarray(x_q8, np.uint8), n_cols))


def _ref_matmul_type(self, w, qtype, x_q8, n_cols):
    """The engine's decode projection (lfm2_matmul_1x4_prequant_mt) for one token."""
    w = np.ascontiguousarray(w, np.uint8)
    out = np.zeros((1, w.shape[0]), np.float32)
    self.lib.ref_matmul_prequant_type(out, w, qtype, w.shape[0], n_cols, np.ascontiguousarray(x_q8, np.uint8))
    return out


_wrap_init(Oracle, _orc_types_init)
_wrap_init(Reference, _ref_types_init)
Oracle.dot_type = _orc_dot_type
Reference.dot_type = _ref_dot_type
Reference.matmul_prequant_type = _ref_matmul_type


def _ref_time_prefill_rows(self, q_rows, k16, v16, pos, n_head_q, kv_mul, kv_dim, max_seq, n_threads, reps=1):
    """Best-of-reps seconds of the reference's per-row prefill attention
    dispatch (lfm2_gqa_heads_worker_task over the heads) for the given rows."""
    q = np.ascontiguousarray(q_rows, np.float32)
    pos = np.ascontiguousarray(pos, np.uint32)
    out = np.zeros((pos.size, n_head_q * 64), np.float32)
    used = _u32(0)
    L = self.lib
    L.ref_time_prefill_rows.restype = C.c_double
    L.ref_time_prefill_rows.argtypes = [_f32p, _u16p, _u16p, _u32p, _f32p, _u32, _u32, _u32, _u32, _u32, _u32,
                                        _u32, C.POINTER(_u32)]
    dt = L.ref_time_prefill_rows(q.reshape(-1), np.ascontiguousarray(k16, np.uint16).reshape(-1),
                                 np.ascontiguousarray(v16, np.uint16).reshape(-1), pos, out, pos.size,
                                 n_head_q, kv_mul, kv_dim, max_seq, n_threads, reps, C.byref(used))
    return dt, int(used.value), out


Reference.time_prefill_rows = _ref_time_prefill_rows
