"""CPU checks of the C-ABI library: it loads, exports every function the
public header declares, builds bit-identical RoPE tables, and rejects bad
arguments with the documented status before touching a device."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import laii_amd as la
from laii_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lfm_attn.h")

E_INVALID, E_RANGE, E_UNSUPPORTED = -1, -2, -3
FAKE = 4096  # never dereferenced: validation rejects the call first


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lfm_(?:attn|hip)_\w+)\s*\(", text)))


def test_header_symbols_exported():
    names = header_functions()
    assert len(names) >= 20
    lib = la.load()
    syms = subprocess.run(["nm", "-D", "--defined-only", la.LIB_PATH], capture_output=True,
                          text=True, check=True).stdout
    for n in names:
        assert re.search(rf"\bT {n}$", syms, flags=re.M), f"{n} not exported"
        assert hasattr(lib, n)
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_no_cpu_fallback_symbols():
    """The product library must not carry a CPU attention path."""
    syms = subprocess.run(["nm", "-D", la.LIB_PATH], capture_output=True, text=True).stdout
    assert "orc_" not in syms and "ref_" not in syms.replace("_ref", "")


def test_device_count_without_gpu():
    n = la.device_count()
    assert n >= 0


def test_status_strings():
    lib = la.load()
    for st in (0, -1, -2, -3, -4, -5):
        assert lib.lfm_attn_status_string(st)


def test_rope_lut_lfm2_bit_exact(orc):
    for hd, base in ((64, 1e6), (64, 1e4), (128, 1e6), (16, 1e6)):
        c, s = la.rope_lut_lfm2(1500, hd, base)
        oc, os_ = orc.rope_lut_lfm2(1500, hd, base)
        assert np.array_equal(c, oc) and np.array_equal(s, os_)


def test_rope_lut_lfm3_bit_exact(orc, ref):
    rf = np.array([1.0] * 32 + [1e30] * 32, np.float32)
    for args in ((128, 128, 1e6, rf), (128, 128, 1e4, None), (128, 64, 1e6, None),
                 (64, 64, 1e6, np.array([2.0, 0.0, -1.0, 1e10] * 8, np.float32))):
        c, s = la.rope_lut_lfm3(700, *args)
        rc, rs = ref.rope_lut_lfm3(700, *args)
        oc, os_ = orc.rope_lut_lfm3(700, *args)
        assert np.array_equal(c, rc) and np.array_equal(s, rs)
        assert np.array_equal(c, oc) and np.array_equal(s, os_)


def test_rope_row_gen1_bit_exact(ref_gen1):
    """The Gen-1 rotation row equals the angles the reference's lfm_rope_neox
    computes per call (src/lfm_forward.c:97-111): its rotation of (1, 0)
    pairs, bit for bit, over head dims and positions past 2^16."""
    for hd in (16, 64, 96, 128):
        for pos in (0, 1, 5, 777, 8191, 32767, 100003):
            c, s = la.rope_row_gen1(hd, pos, 1e6)
            rc, rs = ref_gen1.rope_row(hd, pos, 1e6)
            assert np.array_equal(c, rc) and np.array_equal(s, rs), (hd, pos)
    c, s = la.rope_row_gen1(64, 0, 1e4)
    assert np.all(c == 1.0) and np.all(s == 0.0)


def test_rejections_before_launch():
    lib = la.load()
    # A1: null pointer, kv_dim inconsistent with n_head_q / kv_mul, kv_mul not dividing
    assert lib.lfm_hip_online_gqa_f16(None, FAKE, FAKE, FAKE, 16, 2, 512, 5, 0.125, None) == E_INVALID
    assert lib.lfm_hip_online_gqa_f16(FAKE, FAKE, FAKE, FAKE, 16, 2, 256, 5, 0.125, None) == E_INVALID
    assert lib.lfm_hip_online_gqa_f16(FAKE, FAKE, FAKE, FAKE, 16, 3, 384, 5, 0.125, None) == E_INVALID
    # A2: pos outside the cache, head_dim not a multiple of 8
    assert lib.lfm_hip_gqa_heads(FAKE, None, None, FAKE, FAKE, FAKE, 8, 2, 64, 256, 100, 100, 0.125,
                                 None) == E_RANGE
    assert lib.lfm_hip_gqa_heads(FAKE, None, None, FAKE, FAKE, FAKE, 8, 2, 12, 48, 100, 5, 0.125,
                                 None) == E_INVALID
    assert lib.lfm_hip_gqa_heads(FAKE, None, None, None, FAKE, FAKE, 8, 2, 64, 256, 100, 5, 0.125,
                                 None) == E_INVALID
    # A3: window larger than its ring, linear rows beyond the cache, B == 0
    assert lib.lfm_hip_lfm3_online_gqa_f16_dispatch(FAKE, None, FAKE, FAKE, FAKE, 1, 10, 300, 264,
                                                    16, 4, 128, None) == E_INVALID
    assert lib.lfm_hip_lfm3_online_gqa_f16_dispatch(FAKE, None, FAKE, FAKE, FAKE, 4, 4094, 0, 4096,
                                                    16, 4, 128, None) == E_RANGE
    assert lib.lfm_hip_lfm3_online_gqa_f16_dispatch(FAKE, None, FAKE, FAKE, FAKE, 0, 0, 0, 4096,
                                                    16, 4, 128, None) == E_INVALID
    # varlen: heads not grouped evenly, odd head_dim
    assert lib.lfm_hip_gqa_f16_varlen(FAKE, None, 0, FAKE, FAKE, FAKE, FAKE, 4, 1, 0, 30, 8, 64, 0,
                                      0, 0.125, None) == E_INVALID
    assert lib.lfm_hip_gqa_f16_varlen(FAKE, None, 0, FAKE, FAKE, FAKE, FAKE, 4, 1, 0, 32, 8, 60, 0,
                                      0, 0.125, None) == E_INVALID
    # Gen-1 step: position past the cache, odd head grouping; fused step: a
    # window whose later rows would overwrite earlier rows' keys
    assert lib.lfm_hip_gen1_gqa_step(FAKE, FAKE, FAKE, None, None, FAKE, FAKE, FAKE, 10, 10, 4, 2, 16, 1e-5,
                                     FAKE, FAKE, None) == E_RANGE
    assert lib.lfm_hip_gen1_gqa_step(FAKE, FAKE, FAKE, None, None, FAKE, FAKE, FAKE, 1, 10, 6, 4, 16, 1e-5,
                                     FAKE, FAKE, None) == E_INVALID
    assert lib.lfm_hip_gqa_f16_step(FAKE, FAKE, FAKE, None, 1, FAKE, FAKE, FAKE, FAKE, 1, 8, 0, 16, 4, 128, 256,
                                    260, 0.088, None, None, 1e-5, FAKE, FAKE, 0, None) == E_INVALID
    # prologue forms other than FAST (0) and TABLE (1)
    assert lib.lfm_hip_gqa_f16_step(FAKE, FAKE, FAKE, None, 1, FAKE, FAKE, FAKE, FAKE, 1, 1, 0, 16, 4, 128, 0,
                                    0, 0.088, None, None, 1e-5, FAKE, FAKE, 2, None) == E_INVALID
    # LFM3 prefill: K/V buffer starting after the first row's window start
    # (row 0 at 1000 with window 256 needs position 745), with no window a
    # buffer not starting at 0, head_dim 96, heads not grouped evenly
    f = lib.lfm_hip_lfm3_prefill_f16
    assert f(FAKE, FAKE, FAKE, None, 1, FAKE, 1, 64, 1000, 746, 0, 256, 16, 4, 128, 0.088, None) == E_INVALID
    assert f(FAKE, FAKE, FAKE, None, 1, FAKE, 1, 64, 1000, 1, 0, 0, 16, 4, 128, 0.088, None) == E_INVALID
    assert f(FAKE, FAKE, FAKE, None, 1, FAKE, 1, 64, 1000, 745, 0, 256, 32, 8, 96, 0.102, None) == E_UNSUPPORTED
    assert f(FAKE, FAKE, FAKE, None, 1, FAKE, 1, 64, 0, 0, 0, 0, 12, 8, 128, 0.088, None) == E_INVALID
    # sequences whose buffers would overlap (stride below the rows x kv_dim)
    assert f(FAKE, FAKE, FAKE, None, 1, FAKE, 2, 64, 0, 0, 64 * 512 - 8, 0, 16, 4, 128, 0.088, None) == E_INVALID
    assert lib.lfm_hip_prefill_f16(FAKE, FAKE, FAKE, FAKE, 1, 8, 0, 0, 8, 2, 128, 0.1, None) == E_UNSUPPORTED
    # prologue
    assert lib.lfm_hip_qk_norm_rope(FAKE, None, 4, 63, None, 1e-5, FAKE, FAKE, 0, 0, None) == E_INVALID
    assert lib.lfm_hip_qk_norm_rope(FAKE, None, 4, 64, None, 1e-5, FAKE, FAKE, 0, -1, None) == E_INVALID
    assert lib.lfm_hip_qkv_prologue(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 1, 16, 4, 128, None, None,
                                    1e-5, FAKE, FAKE, 300, 264, 0, None) == E_INVALID
    assert lib.lfm_hip_qkv_prologue(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 1, 16, 4, 128, None, None,
                                    1e-5, FAKE, FAKE, 0, 0, 7, None) == E_INVALID
    out5 = (C.c_uint32 * 5)()
    assert lib.lfm_attn_seg_plan(5, 300, 264, out5) == E_INVALID
    # peak probes: null, unaligned or empty inputs
    assert lib.lfm_hip_probe_read(None, 1 << 20, FAKE, 8, None) == E_INVALID
    assert lib.lfm_hip_probe_read(FAKE + 4, 1 << 20, FAKE, 8, None) == E_INVALID
    assert lib.lfm_hip_probe_read(FAKE, 8, FAKE, 8, None) == E_INVALID
    assert lib.lfm_hip_probe_mfma(None, 8, 16, None) == E_INVALID
    assert lib.lfm_hip_probe_mfma(FAKE, 8, 0, None) == E_INVALID


def test_context_rejects_bad_geometry():
    """Geometry is validated before any device call."""
    import ctypes as C
    from laii_amd._lib import Geom
    lib = la.load()
    g = Geom()
    g.n_layers, g.n_head_q, g.n_head_kv, g.head_dim, g.max_seq = 1, 30, 8, 64, 128
    h = C.c_void_p()
    assert lib.lfm_attn_ctx_create(C.byref(h), C.byref(g)) == E_INVALID  # 30 % 8 != 0
    g.n_head_q, g.head_dim = 32, 60
    assert lib.lfm_attn_ctx_create(C.byref(h), C.byref(g)) == E_INVALID  # head_dim % 8
    g.head_dim = 128
    swa = (C.c_uint8 * 1)(1)
    g.layer_is_swa = C.cast(swa, C.POINTER(C.c_uint8))
    g.sliding_window, g.swa_cap = 256, 200
    assert lib.lfm_attn_ctx_create(C.byref(h), C.byref(g)) == E_INVALID  # window > ring
    g.swa_cap = 262
    assert lib.lfm_attn_ctx_create(C.byref(h), C.byref(g)) == E_INVALID  # 8-row steps need window + 7
    g.layer_is_swa = None
    g.prologue = 1
    g.lfm3 = 1
    assert lib.lfm_attn_ctx_create(C.byref(h), C.byref(g)) == E_INVALID  # LFM3 takes the FAST prologue only
    g.lfm3, g.prologue = 0, 2
    assert lib.lfm_attn_ctx_create(C.byref(h), C.byref(g)) == E_INVALID  # no such prologue form
    assert lib.lfm_attn_ctx_forward(None, 0, 0, 1, FAKE, FAKE, FAKE, None, FAKE) == E_INVALID


def test_shift_sinks_validation_before_launch():
    """Sink-shift entry points: no-op cases return OK with the position kept,
    bad arguments are rejected, all before any device access."""
    lib = la.load()
    ptrs = (C.c_void_p * 2)(FAKE, FAKE)
    nkv = (C.c_uint32 * 2)(8, 8)
    kinds = (C.c_uint8 * 2)(1, 2)
    p = C.c_uint32(10)
    shift2 = lib.lfm_hip_kv_cache_shift_sinks
    shift3 = lib.lfm_hip_lfm3_kv_cache_shift_sinks
    assert shift2(ptrs, ptrs, 2, nkv, 64, FAKE, FAKE, 100, C.byref(p), 4, 8, None) == 0
    assert p.value == 10                                     # pos <= n_sink + n_discard
    p.value = 50
    assert shift2(ptrs, ptrs, 2, nkv, 64, FAKE, FAKE, 100, C.byref(p), 4, 0, None) == 0
    assert p.value == 50                                     # n_discard == 0
    assert shift2(ptrs, ptrs, 2, nkv, 128, FAKE, FAKE, 100, C.byref(p), 4, 8, None) == 0
    assert p.value == 50                                     # LFM2 shifts head_dim 64 only
    assert shift2(ptrs, ptrs, 2, nkv, 64, FAKE, FAKE, 100, None, 4, 8, None) == E_INVALID
    p.value = 300
    assert shift2(ptrs, ptrs, 2, nkv, 64, FAKE, FAKE, 100, C.byref(p), 4, 150, None) == E_RANGE
    assert shift2(None, ptrs, 2, nkv, 64, FAKE, FAKE, 400, C.byref(p), 4, 150, None) == E_INVALID
    odd = (C.c_void_p * 2)(FAKE + 2, FAKE)                   # misaligned cache
    assert shift2(odd, ptrs, 2, nkv, 64, FAKE, FAKE, 400, C.byref(p), 4, 150, None) == E_INVALID
    assert p.value == 300
    # LFM3: rows of either table too few -> no-op; head_dim 72 unsupported; window > ring
    assert shift3(ptrs, ptrs, 2, nkv, kinds, 128, FAKE, FAKE, 100, FAKE, FAKE, 400, 16, 24,
                  C.byref(p), 4, 150, None) == 0 and p.value == 300
    assert shift3(ptrs, ptrs, 2, nkv, kinds, 72, FAKE, FAKE, 400, FAKE, FAKE, 400, 16, 24,
                  C.byref(p), 4, 150, None) == -3
    assert shift3(ptrs, ptrs, 2, nkv, kinds, 128, FAKE, FAKE, 400, FAKE, FAKE, 400, 32, 24,
                  C.byref(p), 4, 150, None) == E_INVALID
    assert shift3(ptrs, ptrs, 2, nkv, kinds, 128, None, FAKE, 400, FAKE, FAKE, 400, 16, 24,
                  C.byref(p), 4, 150, None) == E_INVALID
    assert p.value == 300
    assert lib.lfm_attn_ctx_shift_sinks(None, C.byref(p), 4, 8) == E_INVALID


def test_quant_matmul_validation_before_launch():
    """Q8_K / Q4_K entry points: empty work is OK, other bad arguments are
    rejected before any device access."""
    lib = la.load()
    q8, mm = lib.lfm_hip_quantize_q8_K, lib.lfm_hip_matmul_q4_K
    assert q8(None, None, 0, 256, None) == 0                  # nothing to do
    assert q8(FAKE, None, 1, 256, None) == E_INVALID
    assert q8(FAKE, FAKE, 1, 300, None) == E_UNSUPPORTED      # n_cols % 256
    assert q8(FAKE + 2, FAKE, 1, 256, None) == E_INVALID      # misaligned x
    assert mm(None, None, 0, 256, None, 1, None) == 0
    assert mm(FAKE, FAKE, 4, 256, None, 1, None) == E_INVALID
    assert mm(FAKE, FAKE, 4, 384, FAKE, 1, None) == E_UNSUPPORTED
    assert mm(FAKE, FAKE + 4, 4, 256, FAKE, 1, None) == E_INVALID  # w not 16-byte aligned
    assert mm(FAKE, FAKE, 4, 256, FAKE + 2, 1, None) == E_INVALID  # x_q8 not 4-byte aligned


def test_matmul_prequant_validation_before_launch():
    lib = la.load()
    f = lib.lfm_hip_matmul_prequant
    assert f(FAKE, FAKE, 12, 0, 2048, FAKE, 1, None) == 0           # nothing to do
    assert f(None, FAKE, 12, 8, 2048, FAKE, 1, None) == E_INVALID
    for t in (3, 6, 9, 10, 11, 15, 16, 20, 30):                       # no kernel for these types
        assert f(FAKE, FAKE, t, 8, 2048, FAKE, 1, None) == E_UNSUPPORTED
    assert f(FAKE, FAKE, 2, 8, 2000, FAKE, 1, None) == E_UNSUPPORTED  # n_cols % 256
    assert f(FAKE, FAKE + 8, 13, 8, 2048, FAKE, 1, None) == E_INVALID  # Q5_K rows 16-byte aligned
    assert f(FAKE, FAKE + 4, 23, 8, 2048, FAKE, 1, None) == E_INVALID  # IQ4_XS 8-byte aligned
    assert f(FAKE, FAKE + 1, 8, 8, 2048, FAKE, 1, None) == E_INVALID   # Q8_0 2-byte aligned


def test_qkv_fused_validation_before_launch():
    lib = la.load()
    f = lib.lfm_hip_gqa_qkv_fused
    t = (C.c_uint32 * 4)(12, 12, 14, 12)
    bad = (C.c_uint32 * 4)(12, 12, 10, 12)  # Q2_K: no kernel here
    args = lambda types, cols=2048, wv=FAKE: (FAKE, FAKE, FAKE, None, FAKE, FAKE, wv, None, types, 8, 8, 8,
                                              4, cols, FAKE, 1, None)
    assert f(*args(None)) == E_INVALID
    assert f(*args(bad)) == E_UNSUPPORTED
    assert f(*args(t, cols=300)) == E_UNSUPPORTED
    assert f(*args(t, wv=FAKE + 1)) == E_INVALID            # Q6_K rows need 2-byte alignment
    assert f(FAKE, FAKE, FAKE, None, FAKE + 8, FAKE, FAKE, None, t, 8, 8, 8, 0, 2048, FAKE, 1,
             None) == E_INVALID                             # Q4_K rows need 16-byte alignment


def test_cache_entry_points_validate_without_device():
    """The persistence entry points reject a missing context / output before
    any device work (the context itself needs a GPU)."""
    lib = la.load()
    m = _lib.CacheModelC()
    tok = (C.c_uint32 * 4)(1, 2, 3, 4)
    matched = C.c_uint32(7)
    assert lib.lfm_attn_ctx_cache_save(None, b"/tmp/x", C.byref(m), tok, 4, None, None) == E_INVALID
    assert lib.lfm_attn_ctx_cache_load_prefix(None, b"/tmp/x", C.byref(m), tok, 4, None, None,
                                              C.byref(matched)) == E_INVALID
    assert matched.value == 0
    assert lib.lfm_attn_ctx_cache_load_prefix(None, b"/tmp/x", C.byref(m), tok, 4, None, None,
                                              None) == E_INVALID
    n = C.c_size_t(0)
    assert lib.lfm_attn_ctx_swa_slab_bytes(None, C.byref(n)) == E_INVALID
    assert lib.lfm_attn_ctx_swa_slab_save(None, FAKE) == E_INVALID
    assert lib.lfm_attn_ctx_swa_slab_restore(None, FAKE) == E_INVALID
    assert lib.lfm_attn_status_string(-6) == b"file could not be written"
