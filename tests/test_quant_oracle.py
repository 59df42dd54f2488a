"""Q8_K activations and Q4_K x Q8_K projections (the `wo` / QKV rows beside
the attention path): pins of the oracle restatement (orc_quantize_q8_K,
orc_dot_q4_K_q8_K, orc_matmul_q4_K).

- Bit-exact against the reference's own kernels compiled from source:
  lfm2_quantize_row_q8_K_avx2_cpuid (tools/lfm2_cpuid_quants.c:585-635) and
  lfm2_vec_dot_q4_K_q8_K_avx2 (include/lfm2_simd_avx2.h:364-412).
- Within fp32 rounding of the engine's entry points, whose 1x4 kernels fuse
  the per-block combination into FMAs on AVX-VNNI hosts
  (tools/lfm2_cpuid_quants.c:1189-1250): lfm2_matmul_1x4_prequant_mt and
  lfm2_matmul_batch_avx2_mt.
- Against the float64 closed form of the GGUF Q4_K / Q8_K formats (weights
  d*sc*q - dmin*m, activations d8*q8), and round-half-even on exact ties.

Weight patterns mirror tests/test_decode_1x4.c:122-160, 195-225 and
tests/test_cpuid_quants.c:69-112 of the reference."""
import numpy as np
import pytest

from helpers import (q4k_dequant, q4k_pattern, q4k_random, q6k_dequant, q6k_random, q8k_dequant, q_dequant,
                     q_random)


def test_quantize_matches_reference_test_inputs(orc, ref):
    # tests/test_cpuid_quants.c:72-82 inputs
    i = np.arange(2048, dtype=np.float32)
    x = np.sin(i * np.float32(0.031)) * np.where(i % 2 == 0, np.float32(2.5), np.float32(-1.8))
    assert np.array_equal(orc.quantize_q8_K(x[None]), ref.quantize_q8_K(x[None]))
    z = np.zeros((1, 2048), np.float32)
    qz = orc.quantize_q8_K(z)
    assert not qz.any() and np.array_equal(qz, ref.quantize_q8_K(z))


@pytest.mark.parametrize("seed,scale", [(0, 1.0), (1, 1e-3), (2, 300.0), (3, 1.0)])
def test_quantize_matches_reference_random(orc, ref, seed, scale):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((5, 1024)) * scale).astype(np.float32)
    if seed == 3:
        x[2, 256:512] = 0.0          # one all-zero block
        x[4, :256] = np.float32(7.0)  # constant block: every value is max|x|
    assert np.array_equal(orc.quantize_q8_K(x), ref.quantize_q8_K(x))


def test_quantize_rounds_half_to_even(orc, ref):
    """max|x| = 127 makes 127/max|x| exactly 1, so x*iscale = x: ties round to
    even as the AVX2 cvtps_epi32 does (the scalar variant's roundf would send
    2.5 to 3)."""
    x = np.zeros((1, 256), np.float32)
    vals = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5, 3.49, -3.51], np.float32)
    x[0, :vals.size] = vals
    x[0, 255] = 127.0
    q = orc.quantize_q8_K(x)
    assert np.array_equal(q, ref.quantize_q8_K(x))
    assert q[0, :4].view(np.float32)[0] == np.float32(1.0)
    qs = q[0, 4:260].view(np.int8)
    assert list(qs[:vals.size]) == [0, 2, 2, 0, -2, -2, 126, -126, 3, -4]
    bsums = q[0, 260:292].view(np.int16)
    assert bsums[0] == sum([0, 2, 2, 0, -2, -2, 126, -126, 3, -4])
    assert bsums[15] == 127


def test_dequantized_activations_within_half_step(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 768)).astype(np.float32)
    q = orc.quantize_q8_K(x)
    xr, d = q8k_dequant(q, 768)
    step = np.repeat(d, 256, axis=1)
    assert np.all(np.abs(xr - x) <= 0.5 * step * (1 + 1e-6))


@pytest.mark.parametrize("case", ["1x4_test", "gemm_test", "qkv_q", "random"])
def test_dot_matches_reference_1x1(orc, ref, case):
    n_cols = 1024 if case == "1x4_test" else 2048
    nb = n_cols // 256
    if case == "random":
        w = q4k_random(np.random.default_rng(5), 12, n_cols)
        x = np.random.default_rng(6).standard_normal(n_cols).astype(np.float32)
    else:
        d, dmin, a, b, c, e = {"1x4_test": (0x2A00, 0x2400, 7, 3, 11, 17),
                               "gemm_test": (0x2C00, 0x2200, 1, 2, 3, 5),
                               "qkv_q": (0x2A00, 0x2200, 1, 3, 5, 7)}[case]
        w = q4k_pattern(16, nb, d, dmin, a, b, c, e)
        x = np.sin(np.arange(n_cols, dtype=np.float32) * np.float32(0.017))
    xq = ref.quantize_q8_K(x[None])
    for r in range(w.shape[0]):
        got = orc.dot_q4_K(w[r], xq[0], n_cols)
        want = ref.dot_q4_K(w[r], xq[0], n_cols)
        assert np.float32(got).tobytes() == np.float32(want).tobytes(), (r, got, want)


def test_matmul_close_to_engine_decode_projection(orc, ref):
    """lfm2_matmul_1x4_prequant_mt: 4-row kernels (FMA-fused on AVX-VNNI) plus
    1-row tails; 2048 x 2048 is the LFM2-1.2B `wo` shape, 2050 rows leave a
    tail of 2."""
    rng = np.random.default_rng(7)
    for n_rows in (2048, 2050):
        w = q4k_random(rng, n_rows, 2048)
        xq = orc.quantize_q8_K(rng.standard_normal((1, 2048)).astype(np.float32))
        got = orc.matmul_q4_K(w, xq, 2048)
        want = ref.matmul_q4_K_prequant(w, xq, 2048)
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 2e-6 * scale


@pytest.mark.parametrize("B", [1, 3, 8])
def test_matmul_close_to_engine_batch(orc, ref, B):
    """lfm2_matmul_batch_avx2_mt on fp32 tokens (its own quantize step)."""
    rng = np.random.default_rng(B)
    w = q4k_random(rng, 64, 1536)
    x = rng.standard_normal((B, 1536)).astype(np.float32)
    got = orc.matmul_q4_K(w, orc.quantize_q8_K(x), 1536)
    want = ref.matmul_q4_K_batch(w, x)
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()


def test_dot_closed_form(orc):
    """Dequantized weights and activations in float64: the exact value of what
    the integer sums compute; the fp32 combination stays within its rounding."""
    rng = np.random.default_rng(8)
    n_cols = 2048
    w = q4k_random(rng, 32, n_cols)
    x = rng.standard_normal((2, n_cols)).astype(np.float32)
    xq = orc.quantize_q8_K(x)
    wd = q4k_dequant(w, n_cols)
    xd, _ = q8k_dequant(xq, n_cols)
    exact = xd @ wd.T
    got = orc.matmul_q4_K(w, xq, n_cols)
    bound = 1e-5 * (np.abs(xd) @ np.abs(wd).T)
    assert np.all(np.abs(got - exact) <= bound)


def test_planted_scale_unpack_error_breaks_closed_form(orc):
    """A plausible mistake in the 6-bit scale unpacking (taking the high bits of
    sub-blocks 4..7 from byte j instead of j - 4) moves the dequantized dot off
    the oracle's value."""
    rng = np.random.default_rng(9)
    w = q4k_random(rng, 8, 512)
    xq = orc.quantize_q8_K(rng.standard_normal((1, 512)).astype(np.float32))
    xd, _ = q8k_dequant(xq, 512)
    good = xd @ q4k_dequant(w, 512).T
    bad = xd @ q4k_dequant(w, 512, planted_error=True).T
    got = orc.matmul_q4_K(w, xq, 512)
    assert np.abs(got - good).max() < 1e-3 * np.abs(good).max()
    assert np.abs(got - bad).max() > 0.05 * np.abs(good).max()


@pytest.mark.parametrize("seed", [0, 1])
def test_q6K_dot_matches_reference(orc, ref, seed):
    """Q6_K rows (the `wv` type of Q4_K_M files) bit-exact against
    lfm2_vec_dot_q6_K_q8_K_avx2 (include/lfm2_simd_avx2.h:551-634)."""
    rng = np.random.default_rng(seed)
    w = q6k_random(rng, 16, 2048)
    xq = orc.quantize_q8_K(rng.standard_normal((1, 2048)).astype(np.float32))
    for r in range(16):
        got = orc.dot_q6_K(w[r], xq[0], 2048)
        assert np.float32(got).tobytes() == np.float32(ref.dot_q6_K(w[r], xq[0], 2048)).tobytes()


def test_q6K_closed_form(orc):
    rng = np.random.default_rng(3)
    w = q6k_random(rng, 24, 1024)
    xq = orc.quantize_q8_K(rng.standard_normal((3, 1024)).astype(np.float32))
    xd, _ = q8k_dequant(xq, 1024)
    wd = q6k_dequant(w, 1024)
    got = orc.matmul_q(w, 14, xq, 1024)
    assert np.all(np.abs(got - xd @ wd.T) <= 1e-5 * (np.abs(xd) @ np.abs(wd).T))
    assert np.array_equal(orc.matmul_q(q4k_random(rng, 8, 1024), 12, xq, 1024).shape, (3, 8))


TYPES = {2: "Q4_0", 8: "Q8_0", 13: "Q5_K", 23: "IQ4_XS"}


@pytest.mark.parametrize("qtype", sorted(TYPES))
@pytest.mark.parametrize("seed", [0, 1])
def test_other_types_dot_matches_reference(orc, ref, qtype, seed):
    """Q4_0, Q8_0, Q5_K and IQ4_XS rows bit-exact against the reference's AVX2
    1x1 kernels (lfm2_vec_dot_{q4_0,q8_0,q5_K,iq4_xs}_q8_K_avx2), random blocks
    and a zero activation block."""
    rng = np.random.default_rng(seed * 31 + qtype)
    w = q_random(rng, qtype, 12, 2048)
    x = rng.standard_normal((1, 2048)).astype(np.float32)
    if seed == 1:
        x[0, 512:768] = 0.0
    xq = orc.quantize_q8_K(x)
    for r in range(12):
        got = orc.dot_type(w[r], qtype, xq[0], 2048)
        want = ref.dot_type(w[r], qtype, xq[0], 2048)
        assert np.float32(got).tobytes() == np.float32(want).tobytes(), (TYPES[qtype], r, got, want)


@pytest.mark.parametrize("qtype", sorted(TYPES))
def test_other_types_engine_projection(orc, ref, qtype):
    """The engine's decode projection entry (lfm2_matmul_1x4_prequant_mt
    through the CPU kernel table).  Its Q4_0 / Q8_0 1x4 kernels are four 1x1
    calls, so they equal the oracle bit for bit; the Q5_K / IQ4_XS 1x4 kernels
    fuse the per-block combination into FMAs on AVX-VNNI hosts
    (tools/lfm2_cpuid_quants.c:1317-1394), so they agree within fp32 rounding."""
    rng = np.random.default_rng(qtype)
    w = q_random(rng, qtype, 66, 1536)
    xq = orc.quantize_q8_K(rng.standard_normal((1, 1536)).astype(np.float32))
    got = orc.matmul_q(w, qtype, xq, 1536)
    want = ref.matmul_prequant_type(w, qtype, xq, 1536)
    if qtype in (2, 8):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()


@pytest.mark.parametrize("qtype", sorted(TYPES))
def test_other_types_closed_form(orc, qtype):
    """float64 dequantized weights x dequantized activations (format
    definitions in helpers.q_dequant), within fp32 rounding."""
    rng = np.random.default_rng(100 + qtype)
    w = q_random(rng, qtype, 20, 1024)
    xq = orc.quantize_q8_K(rng.standard_normal((2, 1024)).astype(np.float32))
    xd, _ = q8k_dequant(xq, 1024)
    wd = q_dequant(w, qtype, 1024)
    got = orc.matmul_q(w, qtype, xq, 1024)
    assert np.all(np.abs(got - xd @ wd.T) <= 1e-5 * (np.abs(xd) @ np.abs(wd).T) + 1e-30)


def test_reference_test_patterns_q4_0_q8_0(orc, ref):
    """Weights of tests/test_cpuid_quants.c:116-137 (Q4_0: d 0x2E00, qs
    (i*17 + j*31) & 0xFF) and tests/test_simd_kquants.c:118-121 (Q8_0: d
    0x3000, qs (i*7 + j*3) % 127 - 63), activations as there."""
    n_cols = 2048
    i = np.arange(16 * 64)[:, None]
    q40 = np.zeros((16 * 64, 18), np.uint8)
    q40[:, 0:2] = np.array([0x2E00], np.uint16).view(np.uint8)
    q40[:, 2:] = ((i * 17 + np.arange(16)[None] * 31) & 0xFF).astype(np.uint8)
    q80 = np.zeros((16 * 64, 34), np.uint8)
    q80[:, 0:2] = np.array([0x3000], np.uint16).view(np.uint8)
    q80[:, 2:] = (((i * 7 + np.arange(32)[None] * 3) % 127) - 63).astype(np.int8).view(np.uint8)
    xs = {2: np.cos(np.arange(n_cols, dtype=np.float32) * np.float32(0.019)) * np.float32(1.5),
          8: np.sin(np.arange(n_cols, dtype=np.float32) * np.float32(0.017)) * np.float32(1.5)}
    for qtype, w in ((2, q40.reshape(16, -1)), (8, q80.reshape(16, -1))):
        xq = ref.quantize_q8_K(xs[qtype][None])
        for r in range(16):
            assert (np.float32(orc.dot_type(w[r], qtype, xq[0], n_cols)).tobytes() ==
                    np.float32(ref.dot_type(w[r], qtype, xq[0], n_cols)).tobytes())
