"""ctypes binding of laii_amd/liblfm_attn.so (the C-ABI of include/lfm_attn.h).

Loading fails loudly: there is no CPU fallback anywhere in the package.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "liblfm_attn.so")

_u32 = C.c_uint32
_f32 = C.c_float
_int = C.c_int
_vp = C.c_void_p
_sz = C.c_size_t

# prologue forms (LFM_PROLOGUE_* of include/lfm_attn.h)
PROLOGUE_FAST = 0   # lfm2_kernels_fast.c / LFM3: double-angle tables, AVX2 kernels' sum order
PROLOGUE_TABLE = 1  # lfm2_forward.c / lfm2_prefill_batch.c: float-angle table, lfm2_rmsnorm order

# name -> (restype, argtypes); every function declared in include/lfm_attn.h
SIGNATURES = {
    "lfm_attn_status_string": (C.c_char_p, [_int]),
    "lfm_attn_last_error": (C.c_char_p, []),
    "lfm_attn_last_plan": (C.c_char_p, []),
    "lfm_attn_version": (C.c_char_p, []),
    "lfm_attn_set_tuning": (_int, [C.c_char_p, _u32, _u32, _u32, _u32]),
    "lfm_attn_plan_preview": (_int, [_u32, _u32, _u32, _u32, _u32, _u32, _u32, _int, _int, _u32,
                                     C.POINTER(C.c_char_p), C.POINTER(_u32)]),
    "lfm_attn_prefill_plan_preview": (_int, [_u32, _u32, _u32, _u32, _u32, _u32, _u32, C.POINTER(_u32)]),
    "lfm_attn_device_count": (_int, [C.POINTER(_int)]),
    "lfm_attn_set_device": (_int, [_int]),
    "lfm_attn_dev_alloc": (_int, [C.POINTER(_vp), _sz]),
    "lfm_attn_dev_free": (_int, [_vp]),
    "lfm_attn_copy_h2d": (_int, [_vp, _vp, _sz, _vp]),
    "lfm_attn_copy_d2h": (_int, [_vp, _vp, _sz, _vp]),
    "lfm_attn_copy_d2d": (_int, [_vp, _vp, _sz, _vp]),
    "lfm_attn_memset": (_int, [_vp, _int, _sz, _vp]),
    "lfm_attn_stream_sync": (_int, [_vp]),
    "lfm_attn_profile_events": (_int, [_vp, _vp]),
    "lfm_attn_seg_plan": (_int, [_u32, _u32, _u32, C.POINTER(_u32)]),
    "lfm_attn_slot_of": (_u32, [_u32, _u32, _u32]),
    "lfm_attn_rope_lut_lfm2": (_int, [_vp, _vp, _u32, _u32, _f32]),
    "lfm_attn_rope_lut_lfm3": (_int, [_vp, _vp, _u32, _u32, _u32, _f32, _vp, _u32]),
    "lfm_attn_rope_table_lfm2": (_int, [_vp, _vp, _u32, _u32, _f32]),
    "lfm_hip_qk_norm_rope": (_int, [_vp, _vp, _u32, _u32, _vp, _f32, _vp, _vp, _u32, _int, _vp]),
    "lfm_hip_store_fp32_to_fp16": (_int, [_vp, _vp, _u32, _vp]),
    "lfm_hip_quantize_q8_K": (_int, [_vp, _vp, _u32, _u32, _vp]),
    "lfm_hip_matmul_q4_K": (_int, [_vp, _vp, _u32, _u32, _vp, _u32, _vp]),
    "lfm_hip_matmul_prequant": (_int, [_vp, _vp, _u32, _u32, _u32, _vp, _u32, _vp]),
    "lfm_hip_gqa_qkv_fused": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                     _u32, _u32, _vp, _u32, _vp]),
    "lfm_hip_qkv_prologue": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
                                    _vp, _vp, _f32, _vp, _vp, _u32, _u32, _int, _vp]),
    "lfm_hip_online_gqa_f16": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _f32, _vp]),
    "lfm_hip_gqa_heads": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32,
                                 _f32, _vp]),
    "lfm_hip_lfm3_online_gqa_f16_dispatch": (_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                                    _u32, _u32, _u32, _u32, _vp]),
    "lfm_hip_prefill_f16": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, C.c_uint64, _u32, _u32,
                                   _u32, _f32, _vp]),
    "lfm_hip_lfm3_prefill_f16": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _u32, _u32, _u32, _u32, C.c_uint64,
                                        _u32, _u32, _u32, _u32, _f32, _vp]),
    "lfm_hip_gqa_f16_varlen": (_int, [_vp, _vp, _int, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                      _u32, _u32, _u32, _u32, _f32, _vp]),
    "lfm_attn_rope_row_gen1": (_int, [_vp, _vp, _u32, _u32, _f32]),
    "lfm_hip_gen1_gqa_step": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _f32,
                                     _vp, _vp, _vp]),
    "lfm_hip_gqa_f16_step": (_int, [_vp, _vp, _vp, _vp, _int, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                    _u32, _u32, _u32, _u32, _f32, _vp, _vp, _f32, _vp, _vp, _int, _vp]),
    "lfm_hip_gqa_f16_varlen_noalloc": (_int, [_vp, _vp, _int, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                              _u32, _u32, _u32, _u32, _f32, _vp]),
    "lfm_hip_kv_cache_shift_sinks": (_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _u32,
                                            C.POINTER(_u32), _u32, _u32, _vp]),
    "lfm_hip_lfm3_kv_cache_shift_sinks": (_int, [_vp, _vp, _u32, _vp, _vp, _u32, _vp, _vp, _u32,
                                                 _vp, _vp, _u32, _u32, _u32, C.POINTER(_u32),
                                                 _u32, _u32, _vp]),
}



class Geom(C.Structure):
    """lfm_attn_geom of include/lfm_attn.h."""
    _fields_ = [("n_layers", _u32), ("n_head_q", _u32), ("n_head_kv", _u32), ("head_dim", _u32),
                ("max_seq", _u32), ("sliding_window", _u32), ("swa_cap", _u32),
                ("layer_is_swa", C.POINTER(C.c_uint8)), ("eps", _f32), ("rope_base", _f32),
                ("rope_base_swa", _f32), ("rope_dim", _u32), ("rope_freqs", C.POINTER(_f32)),
                ("n_rope_freqs", _u32), ("lfm3", _int), ("prologue", _int)]


class CacheModelC(C.Structure):
    """lfm_attn_cache_model of include/lfm_attn.h."""
    _fields_ = [("model_fingerprint", C.c_uint64), ("n_model_layers", _u32), ("n_embd", _u32),
                ("n_head_q", _u32), ("shortconv_l_cache", _u32),
                ("ctx_layer", C.POINTER(C.c_int32))]


SIGNATURES.update({
    "lfm_hip_fnv1a64": (_int, [_vp, C.c_size_t, C.c_uint64, C.POINTER(C.c_uint64), _vp]),
    "lfm_hip_probe_read": (_int, [_vp, C.c_uint64, _vp, _u32, _vp]),
    "lfm_hip_probe_mfma": (_int, [_vp, _u32, _u32, _vp]),
    "lfm_attn_ctx_cache_save": (_int, [_vp, C.c_char_p, C.POINTER(CacheModelC), _vp, _u32, _vp, _vp]),
    "lfm_attn_ctx_cache_load_prefix": (_int, [_vp, C.c_char_p, C.POINTER(CacheModelC), _vp, _u32, _vp,
                                              _vp, C.POINTER(_u32)]),
    "lfm_attn_ctx_swa_slab_bytes": (_int, [_vp, C.POINTER(C.c_size_t)]),
    "lfm_attn_ctx_swa_slab_save": (_int, [_vp, _vp]),
    "lfm_attn_ctx_swa_slab_restore": (_int, [_vp, _vp]),
    "lfm_attn_ctx_create": (_int, [C.POINTER(_vp), C.POINTER(Geom)]),
    "lfm_attn_ctx_destroy": (None, [_vp]),
    "lfm_attn_ctx_set_norms": (_int, [_vp, _u32, _vp, _vp]),
    "lfm_attn_ctx_forward": (_int, [_vp, _u32, _u32, _u32, _vp, _vp, _vp, _vp, _vp]),
    "lfm_attn_ctx_prefill": (_int, [_vp, _u32, _u32, _u32, _vp, _vp, _vp, _vp, _vp]),
    "lfm_attn_ctx_kv_export": (_int, [_vp, _u32, _u32, _u32, _vp, _vp]),
    "lfm_attn_ctx_kv_import": (_int, [_vp, _u32, _u32, _u32, _vp, _vp]),
    "lfm_attn_ctx_kv_device": (_int, [_vp, _u32, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_u32)]),
    "lfm_attn_ctx_shift_sinks": (_int, [_vp, C.POINTER(_u32), _u32, _u32]),
})

_lock = threading.Lock()
_lib = None


class LfmAttnError(RuntimeError):
    def __init__(self, status: int, where: str, detail: str = ""):
        self.status = status
        super().__init__(f"{where}: status {status} ({detail})")


def load() -> C.CDLL:
    """Load the native library (built by laii_amd.build / __graft_entry__.build)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(status: int, where: str) -> None:
    if status != 0:
        lib = load()
        raise LfmAttnError(status, where, lib.lfm_attn_status_string(status).decode() + " " +
                           lib.lfm_attn_last_error().decode())
