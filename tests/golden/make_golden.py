"""Write tests/golden/golden_ref.npz: outputs of the reference's own CPU
kernels (compiled from /root/reference by oracle/Makefile into
oracle/_ref/libref_attn.so) on the inputs of the reference's own tests.

Run in a container that has /root/reference:
    make -C oracle ref && python tests/golden/make_golden.py

Cases (inputs reproduced from the reference tests, outputs from the reference):
  qk_lfm2   tests/test_kernels_fast.c:121-173  16 heads d64 pos 42, sinf/cosf inputs
  qk_lfm3   tests/test_lfm3.c:104-168          4 heads d128 pos 17, partial RoPE
  a1        tests/test_kernels_fast.c:175-236  16q/4kv d64 seq 128 pos 37
  a2_f32    same inputs through the FP32 two-pass branch
  a2_one    tests/test_optimizations.c:324-421 1 head d64 seq 32 (fp16 branch)
  a3_wrap   tests/test_lfm3.c:170-251          8q/2kv d128 win 16 cap 24, pos 0..41
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.bindings import Reference  # noqa: E402


def f32(x):
    return np.asarray(x, np.float32)


def main():
    ref = Reference()
    assert ref.has_avx2, "the reference's production path is AVX2+F16C"
    g = {}

    # qk_lfm2
    cos, sin = ref.rope_lut_lfm2(128, 64, 1e6)
    q = np.sin(np.arange(1024, dtype=np.float32) * np.float32(0.04)).astype(np.float32)
    nw = (np.float32(1.0) + np.float32(0.05) * np.cos(np.arange(64, dtype=np.float32))).astype(np.float32)
    g["qk_lfm2_in"], g["qk_lfm2_w"] = q, nw
    g["qk_lfm2_out"] = ref.qk_norm_rope(q, 16, 64, nw, 1e-5, cos, sin, 42)
    g["qk_lfm2_k16"] = ref.qk_norm_rope(q, 16, 64, nw, 1e-5, cos, sin, 42, store_f16=True)

    # qk_lfm3 (partial RoPE)
    rf = np.array([1.0] * 32 + [1e30] * 32, np.float32)
    nw3 = (np.float32(1.0) + np.float32(0.01) * (np.arange(128) % 17).astype(np.float32)).astype(np.float32)
    c3, s3 = ref.rope_lut_lfm3(64, 128, 128, 1e6, rf)
    v3 = np.sin(np.arange(512, dtype=np.float32) * np.float32(0.13)).astype(np.float32)
    ref._force_lfm3 = True
    g["qk_lfm3_in"], g["qk_lfm3_w"], g["qk_lfm3_rf"] = v3, nw3, rf
    g["qk_lfm3_out"] = ref.qk_norm_rope(v3, 4, 128, nw3, 1e-5, c3, s3, 17)
    g["qk_lfm3_k16"] = ref.qk_norm_rope(v3, 4, 128, nw3, 1e-5, c3, s3, 17, store_f16=True)
    ref._force_lfm3 = False

    # a1 / a2_f32
    nq, nkv, hd, seq, pos = 16, 4, 64, 128, 37
    kv = nkv * hd
    qa = np.cos(np.arange(nq * hd, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    i = np.arange(seq * kv, dtype=np.float32)
    kf, vf = np.sin(i * np.float32(0.01)).astype(np.float32), np.cos(i * np.float32(0.02)).astype(np.float32)
    k16, v16 = ref.store_f16(kf), ref.store_f16(vf)
    g["a1_q"], g["a1_k16"], g["a1_v16"] = qa, k16, v16
    g["a1_out"] = ref.online_gqa_f16(qa, k16, v16, nq, nq // nkv, kv, pos)
    g["a2_f32_out"] = ref.gqa_heads(qa, nq, nq // nkv, hd, kv, seq, pos, k32=kf, v32=vf)

    # a2_one (tests/test_optimizations.c:324-421)
    q1 = f32([np.float32(0.1) * np.float32(i % 7) - np.float32(0.3) for i in range(64)])
    t, d = np.meshgrid(np.arange(32), np.arange(64), indexing="ij")
    k1 = (np.float32(0.05) * ((t + d) % 11).astype(np.float32) - np.float32(0.25)).astype(np.float32)
    v1 = (np.float32(0.08) * ((t * 2 + d) % 13).astype(np.float32) - np.float32(0.4)).astype(np.float32)
    g["a2_one_q"], g["a2_one_k"], g["a2_one_v"] = q1, k1, v1
    g["a2_one_out"] = ref.gqa_heads(q1, 1, 1, 64, 64, 32, 31, k16=ref.store_f16(k1),
                                    v16=ref.store_f16(v1))

    # a3_wrap (tests/test_lfm3.c:170-251)
    nq, nkv, hd, win, cap = 8, 2, 128, 16, 24
    kv = nkv * hd
    k_ring = np.zeros((cap, kv), np.uint16)
    v_ring = np.zeros((cap, kv), np.uint16)
    gate = (np.float32(0.25) + np.float32(0.08) * np.arange(nq, dtype=np.float32)).astype(np.float32)
    outs, rings_k, rings_v, qs = [], [], [], []
    for p in range(42):
        slot = p % cap
        ii = np.arange(kv, dtype=np.float32)
        k_ring[slot] = ref.store_f16(np.float32(0.4) * np.sin((np.float32(p * 19) + ii) * np.float32(0.11)))
        v_ring[slot] = ref.store_f16(np.float32(0.5) * np.cos((np.float32(p * 23) + ii) * np.float32(0.09)))
        qp = (np.float32(0.3) * np.sin((np.float32(p * 13) + np.arange(nq * hd, dtype=np.float32))
                                       * np.float32(0.07))).astype(np.float32)
        outs.append(ref.lfm3_dispatch(qp, gate, k_ring, v_ring, 1, p, win, cap, nq, nkv, hd))
        rings_k.append(k_ring.copy())
        rings_v.append(v_ring.copy())
        qs.append(qp)
    g["a3_gate"] = gate
    g["a3_q"], g["a3_k"], g["a3_v"], g["a3_out"] = (np.stack(qs), np.stack(rings_k),
                                                    np.stack(rings_v), np.stack(outs))
    path = os.path.join(HERE, "golden_ref.npz")
    np.savez_compressed(path, **g)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
