"""GPU parity of the projections beside the attention path:
lfm_hip_quantize_q8_K and lfm_hip_matmul_q4_K against the oracle
(orc_quantize_q8_K / orc_matmul_q4_K, pinned bit-exact to the reference's
lfm2_quantize_row_q8_K_avx2_cpuid and lfm2_vec_dot_q4_K_q8_K_avx2 in
test_quant_oracle.py).  Both are bit-exact: the quantizer's integer outputs
and correctly rounded scale, and the product's exact integer sums combined in
the reference's fp32 order."""
import numpy as np
import pytest

from helpers import parity, q4k_pattern, q4k_random, q6k_random, q_random

pytestmark = pytest.mark.gpu


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def gpu_quantize(la, x):
    x = np.ascontiguousarray(x, np.float32)
    y = la.DeviceArray.zeros((x.shape[0], x.shape[1] // 256 * 292), np.uint8)
    la.quantize_q8_K(dev(la, x), y, x.shape[0], x.shape[1])
    return y.numpy()


def gpu_matmul(la, w, xq, n_cols):
    out = la.DeviceArray.zeros((xq.shape[0], w.shape[0]), np.float32)
    la.matmul_q4_K(out, dev(la, w), w.shape[0], n_cols, dev(la, xq), xq.shape[0])
    return out.numpy()


def test_quantize_reference_test_inputs(gpu, orc):
    i = np.arange(2048, dtype=np.float32)
    x = np.sin(i * np.float32(0.031)) * np.where(i % 2 == 0, np.float32(2.5), np.float32(-1.8))
    assert np.array_equal(gpu_quantize(gpu, x[None]), orc.quantize_q8_K(x[None]))


@pytest.mark.parametrize("seed,rows,cols,scale", [(0, 1, 256, 1.0), (1, 7, 2048, 1e-3),
                                                  (2, 64, 2048, 40.0), (3, 3, 8192, 1.0)])
def test_quantize_bit_exact(gpu, orc, seed, rows, cols, scale):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    if rows > 2:
        x[1, :256] = 0.0                    # all-zero block
        x[2, 256:512] = np.float32(-3.0)    # constant block
    assert np.array_equal(gpu_quantize(gpu, x), orc.quantize_q8_K(x))


def test_quantize_ties_round_half_to_even(gpu, orc):
    x = np.zeros((1, 256), np.float32)
    vals = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float32)
    x[0, :vals.size] = vals
    x[0, 255] = 127.0
    q = gpu_quantize(gpu, x)
    assert np.array_equal(q, orc.quantize_q8_K(x))
    assert list(q[0, 4:4 + vals.size].view(np.int8)) == [0, 2, 2, 0, -2, -2, 126, -126]


@pytest.mark.parametrize("n_rows,n_cols,B", [(4, 1024, 1), (16, 2048, 1), (2048, 2048, 1),
                                             (5, 2304, 3), (130, 1536, 8), (64, 8192, 2),
                                             (1, 256, 64), (2048, 2048, 64),
                                             # int8-MFMA path (16-row tiles, >= 8 tokens):
                                             # super-block rounds of 8 with a remainder,
                                             # ragged token tiles, one super-block
                                             (32, 2304, 17), (48, 512, 100), (16, 256, 8)])
def test_matmul_bit_exact_random(gpu, orc, n_rows, n_cols, B):
    rng = np.random.default_rng(n_rows * 7 + n_cols + B)
    w = q4k_random(rng, n_rows, n_cols)
    x = rng.standard_normal((B, n_cols)).astype(np.float32)
    if n_cols >= 512:
        x[0, 256:512] = 0.0  # a block with d8 == 0 is skipped
    xq = orc.quantize_q8_K(x)
    got = gpu_matmul(gpu, w, xq, n_cols)
    want = orc.matmul_q4_K(w, xq, n_cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("case", ["1x4_test", "gemm_test", "qkv_k", "qkv_v"])
def test_matmul_reference_test_patterns(gpu, orc, case):
    """Weights of the reference's tests (tests/test_decode_1x4.c:122-160,
    195-260), activations sin/cos as there."""
    n_cols = 1024 if case == "1x4_test" else 2048
    d, dmin, a, b, c, e = {"1x4_test": (0x2A00, 0x2400, 7, 3, 11, 17),
                           "gemm_test": (0x2C00, 0x2200, 1, 2, 3, 5),
                           "qkv_k": (0x2B00, 0x2300, 2, 5, 7, 11),
                           "qkv_v": (0x2C00, 0x2400, 3, 7, 11, 13)}[case]
    w = q4k_pattern(512, n_cols // 256, d, dmin, a, b, c, e)
    x = np.cos(np.arange(n_cols, dtype=np.float32) * np.float32(0.031))[None]
    xq = orc.quantize_q8_K(x)
    got = gpu_matmul(gpu, w, xq, n_cols)
    want = orc.matmul_q4_K(w, xq, n_cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_attention_output_to_wo_projection(gpu, orc):
    """Decode step of an LFM2 attention layer (16q/8kv, d64, pos 700): A1
    attention on the device, its output quantized to Q8_K (the reference's
    per-4-head side effect), then the 1024 x 1024 `wo` product -- against the
    oracle chain on the same inputs, within the attention tolerance."""
    la = gpu
    rng = np.random.default_rng(11)
    nq, nkv, hd, pos = 16, 8, 64, 700
    q = rng.standard_normal(nq * hd).astype(np.float32)
    k16 = (rng.standard_normal((pos + 1, nkv * hd)) * 0.5).astype(np.float16).view(np.uint16)
    v16 = (rng.standard_normal((pos + 1, nkv * hd)) * 0.5).astype(np.float16).view(np.uint16)
    w = q4k_random(rng, nq * hd, nq * hd)
    xb = la.DeviceArray.zeros(nq * hd, np.float32)
    la.online_gqa_f16(dev(la, q), dev(la, k16), dev(la, v16), xb, nq, nq // nkv, nkv * hd, pos,
                      1.0 / 8.0)
    xq = la.DeviceArray.zeros((1, nq * hd // 256 * 292), np.uint8)
    la.quantize_q8_K(xb, xq, 1, nq * hd)
    out = la.DeviceArray.zeros((1, nq * hd), np.float32)
    la.matmul_q4_K(out, dev(la, w), nq * hd, nq * hd, xq, 1)
    xb_h = xb.numpy()
    # the device chain is bit-exact from its own attention output on
    assert np.array_equal(xq.numpy(), orc.quantize_q8_K(xb_h[None]))
    assert np.array_equal(out.numpy(), orc.matmul_q4_K(w, xq.numpy(), nq * hd))
    # and within tolerance of the oracle's attention
    want_xb = orc.online_gqa_f16(q, k16, v16, nq, nq // nkv, nkv * hd, pos, 1.0 / 8.0)
    parity(xb_h, want_xb, what="attention")
    want = orc.matmul_q4_K(w, orc.quantize_q8_K(want_xb[None]), nq * hd)
    parity(out.numpy(), want, max_abs=2e-3 * max(1.0, float(np.abs(want).max())), what="wo")


@pytest.mark.parametrize("n_rows,n_cols,B", [(8, 256, 1), (512, 2048, 1), (130, 2304, 5), (64, 2048, 64)])
def test_q6K_matmul_bit_exact(gpu, orc, n_rows, n_cols, B):
    """Q6_K rows (210-byte blocks, 2-byte aligned) through the fused entry."""
    la = gpu
    rng = np.random.default_rng(n_rows + B)
    w = q6k_random(rng, n_rows, n_cols)
    xq = orc.quantize_q8_K(rng.standard_normal((B, n_cols)).astype(np.float32))
    out = la.DeviceArray.zeros((B, n_rows), np.float32)
    la.gqa_qkv_fused([out], [dev(la, w)], [la.GGML_Q6_K], [n_rows], n_cols, dev(la, xq), B)
    want = orc.matmul_q(w, 14, xq, n_cols)
    assert np.array_equal(out.numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("B,gate,v_type", [(1, False, 12), (1, True, 14), (8, True, 14), (3, False, 14)])
def test_qkv_fused_lfm2_lfm3_shapes(gpu, orc, B, gate, v_type):
    """LFM2-1.2B Q/K/V (2048 -> 2048 / 512 / 512) and LFM3 with the gate
    (16 rows): every output bit-exact against the oracle row by row, V in
    Q4_K or Q6_K (Q4_K_M files store some `wv` as Q6_K)."""
    la = gpu
    rng = np.random.default_rng(B * 3 + gate)
    n_cols, rows = 2048, [2048, 512, 512] + ([16] if gate else [])
    types = [12, 12, v_type] + ([12] if gate else [])
    ws = [q6k_random(rng, r, n_cols) if t == 14 else q4k_random(rng, r, n_cols)
          for r, t in zip(rows, types)]
    xq = orc.quantize_q8_K(rng.standard_normal((B, n_cols)).astype(np.float32))
    outs = [la.DeviceArray.zeros((B, r), np.float32) for r in rows]
    la.gqa_qkv_fused(outs, [dev(la, w) for w in ws], types, rows, n_cols, dev(la, xq), B)
    for o, w, t in zip(outs, ws, types):
        want = orc.matmul_q(w, t, xq, n_cols)
        assert np.array_equal(o.numpy().view(np.uint32), want.view(np.uint32))


OTHER_TYPES = {2: "Q4_0", 8: "Q8_0", 13: "Q5_K", 23: "IQ4_XS"}


@pytest.mark.parametrize("qtype", sorted(OTHER_TYPES))
@pytest.mark.parametrize("n_rows,n_cols,B", [(8, 256, 1), (2048, 2048, 1), (130, 2304, 5), (64, 2048, 64),
                                             (32, 2304, 17)])
def test_other_types_bit_exact(gpu, orc, qtype, n_rows, n_cols, B):
    """Q4_0, Q8_0, Q5_K and IQ4_XS rows through lfm_hip_matmul_prequant,
    bit-exact against the oracle (pinned to the reference's AVX2 1x1 dots),
    including a zero activation block."""
    la = gpu
    rng = np.random.default_rng(qtype * 1000 + n_rows + B)
    w = q_random(rng, qtype, n_rows, n_cols)
    x = rng.standard_normal((B, n_cols)).astype(np.float32)
    if n_cols >= 512:
        x[0, 256:512] = 0.0
    xq = orc.quantize_q8_K(x)
    out = la.DeviceArray.zeros((B, n_rows), np.float32)
    la.matmul_prequant(out, dev(la, w), qtype, n_rows, n_cols, dev(la, xq), B)
    want = orc.matmul_q(w, qtype, xq, n_cols)
    assert np.array_equal(out.numpy().view(np.uint32), want.view(np.uint32)), OTHER_TYPES[qtype]


@pytest.mark.parametrize("B", [3, 9])
def test_fused_mixed_types(gpu, orc, B):
    """One fused call over four matrices of four different types (Q5_K Q,
    IQ4_XS K, Q8_0 V, Q4_0 gate); at 9 tokens the Q5_K matrix takes the
    int8-MFMA kernel and the rest one dot4 launch."""
    la = gpu
    rng = np.random.default_rng(99 + B)
    n_cols, rows, types = 2048, [2048, 512, 512, 16], [13, 23, 8, 2]
    ws = [q_random(rng, t, r, n_cols) for t, r in zip(types, rows)]
    xq = orc.quantize_q8_K(rng.standard_normal((B, n_cols)).astype(np.float32))
    outs = [la.DeviceArray.zeros((B, r), np.float32) for r in rows]
    la.gqa_qkv_fused(outs, [dev(la, w) for w in ws], types, rows, n_cols, dev(la, xq), B)
    for o, w, t in zip(outs, ws, types):
        assert np.array_equal(o.numpy().view(np.uint32), orc.matmul_q(w, t, xq, n_cols).view(np.uint32))


@pytest.mark.parametrize("qtype", [2, 8])
def test_q4_0_q8_0_reference_patterns(gpu, orc, qtype):
    """Weight patterns of tests/test_cpuid_quants.c:116-137 (Q4_0) and
    tests/test_simd_kquants.c:118-121 (Q8_0)."""
    la = gpu
    n_cols, n_rows = 2048, 64
    i = np.arange(n_rows * 64)[:, None]
    if qtype == 2:
        blk = np.zeros((n_rows * 64, 18), np.uint8)
        blk[:, 0:2] = np.array([0x2E00], np.uint16).view(np.uint8)
        blk[:, 2:] = ((i * 17 + np.arange(16)[None] * 31) & 0xFF).astype(np.uint8)
        x = np.cos(np.arange(n_cols, dtype=np.float32) * np.float32(0.019)) * np.float32(1.5)
    else:
        blk = np.zeros((n_rows * 64, 34), np.uint8)
        blk[:, 0:2] = np.array([0x3000], np.uint16).view(np.uint8)
        blk[:, 2:] = (((i * 7 + np.arange(32)[None] * 3) % 127) - 63).astype(np.int8).view(np.uint8)
        x = np.sin(np.arange(n_cols, dtype=np.float32) * np.float32(0.017)) * np.float32(1.5)
    w = blk.reshape(n_rows, -1)
    xq = orc.quantize_q8_K(x[None])
    out = la.DeviceArray.zeros((1, n_rows), np.float32)
    la.matmul_prequant(out, dev(la, w), qtype, n_rows, n_cols, dev(la, xq), 1)
    assert np.array_equal(out.numpy().view(np.uint32), orc.matmul_q(w, qtype, xq, n_cols).view(np.uint32))
