"""Pins the CPU oracle (oracle/cpu_attn.c) before any GPU result is checked
against it: textbook closed forms in float64, the reference's own test inputs
and tolerances, golden vectors written by the compiled reference
(tests/golden/golden_ref.npz), the PyTorch fixture of the reference
(tests/golden/fixtures_attention.bin), and the compiled reference itself when
it is present.  Planted mistakes (in the oracle's inputs, on the CPU) show
that each check would catch a dropped term, a wrong index or a transposed
operand."""
import os
import struct

import numpy as np
import pytest

from helpers import f16, f16_to_f32, softmax_attention_f64

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLDEN, "golden_ref.npz"), allow_pickle=False)


# ---- A8: fp16 -------------------------------------------------------------------------------

def test_f16_to_f32_all_halves(orc):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = orc.f16_to_f32(h)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan], want[~nan]) and np.all(np.isnan(got[nan]))


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(0)
    hv = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((hv[:-1] + hv[1:]) / 2).astype(np.float32)  # exact ties -> even
    x = np.concatenate([rng.standard_normal(1 << 18).astype(np.float32) * s
                        for s in (1e-7, 1e-5, 1e-2, 1.0, 1e3, 6e4)] +
                       [mids, -mids, np.array([65504, 65519.99, 65520, 1e9, -1e9, 0.0, -0.0,
                                               2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -25, np.inf,
                                               -np.inf], np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16(x), want)


def test_f32_to_f16_matches_f16c(orc, ref):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(1 << 18) * 10.0 ** rng.integers(-8, 5, 1 << 18)).astype(np.float32)
    assert np.array_equal(orc.f32_to_f16(x), ref.store_f16(x))


# ---- A4/A5: RoPE tables and QK-norm ------------------------------------------------------------

def test_rope_lut_closed_form(orc):
    """cos/sin(pos * base^(-2i/d)) in float64, rounded to float32 (<= 1 ulp)."""
    for hd, base in ((64, 1e6), (128, 1e4)):
        c, s = orc.rope_lut_lfm2(4096, hd, base)
        i = np.arange(hd // 2, dtype=np.float64)
        ang = np.arange(4096, dtype=np.float64)[:, None] * np.power(float(np.float32(base)), -(2 * i) / hd)
        for got, want in ((c, np.cos(ang)), (s, np.sin(ang))):
            ulp = np.spacing(np.abs(want).astype(np.float32))
            assert np.all(np.abs(got - want) <= ulp * 1.01 + 1e-30)


def test_rope_lut_matches_reference(orc, ref):
    for hd, base in ((64, 1e6), (64, 1e4), (128, 1e6)):
        assert all(np.array_equal(a, b) for a, b in zip(orc.rope_lut_lfm2(900, hd, base),
                                                        ref.rope_lut_lfm2(900, hd, base)))
    rf = np.array([1.0] * 32 + [1e30] * 32, np.float32)
    assert all(np.array_equal(a, b) for a, b in zip(orc.rope_lut_lfm3(900, 128, 128, 1e6, rf),
                                                    ref.rope_lut_lfm3(900, 128, 128, 1e6, rf)))


def test_partial_rope_identity_pairs(orc):
    """tests/test_lfm3.c:104-126: pairs i >= 32 are the identity (cos 1, sin 0)."""
    rf = np.array([1.0] * 32 + [1e30] * 32, np.float32)
    c, s = orc.rope_lut_lfm3(64, 128, 128, 1e6, rf)
    assert np.all(c[:, 32:] == 1.0) and np.all(s[:, 32:] == 0.0)
    assert not np.all(c[17, :32] == 1.0)
    c2, s2 = orc.rope_lut_lfm3(64, 128, 64, 1e6, None)  # rope_dim 64 -> first 32 pairs rotate
    assert np.all(c2[:, 32:] == 1.0) and np.array_equal(c2[:, :32], c[:, :32])


def _norm_rope_f64(x, n_heads, hd, w, eps, c, s):
    x = x.reshape(n_heads, hd).astype(np.float64)
    if w is not None:
        x = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)
    lo, hi = x[:, :hd // 2], x[:, hd // 2:]
    c, s = c.astype(np.float64), s.astype(np.float64)
    return np.concatenate([lo * c - hi * s, hi * c + lo * s], axis=1).reshape(-1)


def test_qk_norm_rope_closed_form(orc):
    rng = np.random.default_rng(2)
    for hd in (64, 128, 16):
        c, s = orc.rope_lut_lfm2(100, hd, 1e6)
        x = rng.standard_normal(8 * hd).astype(np.float32) * 2
        w = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
        got = orc.qk_norm_rope(x, 8, hd, w, 1e-5, c[77], s[77])
        want = _norm_rope_f64(x, 8, hd, w, 1e-5, c[77], s[77])
        assert np.abs(got - want).max() < 5e-6
        # invariant: the rotation preserves each pair's norm; the RMSNorm fixes the mean square
        g = got.reshape(8, hd).astype(np.float64)
        assert np.allclose((g * g).mean(1), ((x.reshape(8, hd) / np.sqrt((x.reshape(8, hd) ** 2).mean(1, keepdims=True) + 1e-5) * w) ** 2).mean(1), rtol=1e-5)


def test_qk_norm_rope_reference_inputs(orc, gold):
    """tests/test_kernels_fast.c:121-173 (16 heads, d64, pos 42): within 1e-4 of
    the powf/cosf/sinf formula there, and bit-identical to the reference
    kernel's golden output (Q fp32 and the fp16 K store)."""
    q, w = gold["qk_lfm2_in"], gold["qk_lfm2_w"]
    c, s = orc.rope_lut_lfm2(128, 64, 1e6)
    got = orc.qk_norm_rope(q, 16, 64, w, 1e-5, c[42], s[42])
    assert np.array_equal(got.view(np.uint32), gold["qk_lfm2_out"].view(np.uint32))
    want = q.reshape(16, 64).astype(np.float64)
    want = want / np.sqrt((want ** 2).mean(1, keepdims=True) + 1e-5) * w
    i = np.arange(32)
    f = np.power(1e6, -(2.0 * i) / 64)
    cc, ss = np.cos(42 * f), np.sin(42 * f)
    want = np.concatenate([want[:, :32] * cc - want[:, 32:] * ss, want[:, 32:] * cc + want[:, :32] * ss], 1)
    assert np.abs(got - want.reshape(-1)).max() < 1e-4
    k16 = orc.qk_norm_rope(q, 16, 64, w, 1e-5, c[42], s[42], store_f16=True)
    assert np.array_equal(k16, gold["qk_lfm2_k16"])


def test_qk_norm_rope_partial_reference(orc, gold):
    """tests/test_lfm3.c:104-168: d128 partial RoPE, pos 17, 4 heads;
    bit-identical to the reference kernel's golden output."""
    c, s = orc.rope_lut_lfm3(64, 128, 128, 1e6, gold["qk_lfm3_rf"])
    got = orc.qk_norm_rope(gold["qk_lfm3_in"], 4, 128, gold["qk_lfm3_w"], 1e-5, c[17], s[17])
    assert np.array_equal(got.view(np.uint32), gold["qk_lfm3_out"].view(np.uint32))
    k16 = orc.qk_norm_rope(gold["qk_lfm3_in"], 4, 128, gold["qk_lfm3_w"], 1e-5, c[17], s[17],
                           store_f16=True)
    assert np.array_equal(k16, gold["qk_lfm3_k16"])


@pytest.mark.parametrize("hd", [64, 128])
def test_qk_norm_rope_matches_reference_kernels(orc, ref, hd):
    """Bit for bit against the engine's AVX2 kernels (lfm2_qk_norm_rope_avx2
    at d64, lfm3_qk_norm_rope_128_avx2 at d128): the sum of squares in their
    column order and horizontal-sum tree, fmsub/fmadd rotation, RNE store;
    the scalar kernels (double or float sums, separately rounded rotation)
    within 2e-6."""
    rng = np.random.default_rng(4)
    if hd == 64:
        c, s = orc.rope_lut_lfm2(512, 64, 1e6)
    else:
        c, s = orc.rope_lut_lfm3(512, 128, 128, 1e6, np.array([1.0] * 32 + [1e30] * 32, np.float32))
    for trial in range(20):
        x = rng.standard_normal(32 * hd).astype(np.float32) * np.float32(3 if trial % 2 else 0.01)
        w = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        mine = orc.qk_norm_rope(x, 32, hd, w, 1e-5, c[300], s[300])
        assert np.array_equal(mine.view(np.uint32), ref.qk_norm_rope(x, 32, hd, w, 1e-5, c, s, 300).view(np.uint32))
        k_mine = orc.qk_norm_rope(x, 32, hd, w, 1e-5, c[300], s[300], store_f16=True)
        assert np.array_equal(k_mine, ref.qk_norm_rope(x, 32, hd, w, 1e-5, c, s, 300, store_f16=True))
        theirs = ref.qk_norm_rope(x, 32, hd, w, 1e-5, c, s, 300, scalar=True)
        assert np.abs(mine - theirs).max() < 2e-6


def test_qk_norm_rope_order_pins_a_planted_mistake(orc, ref):
    """A sum of squares added in plain sequential order (a plausible
    restatement) is not bit-identical to the AVX2 kernels on these inputs,
    so the bit-exact check above has teeth."""
    rng = np.random.default_rng(9)
    c, s = orc.rope_lut_lfm2(64, 64, 1e6)
    diffs = 0
    for _ in range(20):
        x = rng.standard_normal(16 * 64).astype(np.float32) * 3
        w = (1 + 0.05 * rng.standard_normal(64)).astype(np.float32)
        theirs = ref.qk_norm_rope(x, 16, 64, w, 1e-5, c, s, 33)
        xs = x.reshape(16, 64)
        ss = np.zeros(16, np.float32)
        for i in range(64):
            ss = (ss + xs[:, i] * xs[:, i]).astype(np.float32)
        irms = (np.float32(1.0) / np.sqrt(ss / np.float32(64) + np.float32(1e-5))).astype(np.float32)
        normed = ((xs * irms[:, None]).astype(np.float32) * w).astype(np.float32)
        mine = orc.qk_norm_rope(normed.reshape(-1), 16, 64, None, 1e-5, c[33], s[33])
        diffs += int(np.count_nonzero(mine.view(np.uint32) != theirs.view(np.uint32)))
    assert diffs > 0


# ---- A4, the production LFM2 stacks (lfm2_forward.c, lfm2_prefill_batch.c) ----------------------

def test_rope_table_lfm2_closed_form(orc):
    """The float-angle table: entry (p, i) is cosf / sinf of the float
    product fl(p * freq_i), freq_i = powf(base, -(2i/d)); against float64
    cos / sin of that same float angle (<= 1 ulp), with freq_i within 1 ulp
    of the float64 power.  The double-angle table differs from it past
    position ~1000 by up to ~1e-3 (the float angle's rounding), which is what
    makes the two prologues distinguishable."""
    for hd, base in ((64, 1e6), (64, 1e4), (128, 1e6)):
        c, s = orc.rope_table_lfm2(32768, hd, base)
        i = np.arange(hd // 2)
        freq64 = np.power(float(np.float32(base)), -(2.0 * i) / hd)
        freq = freq64.astype(np.float32)
        # the float angle, rebuilt with the table's own frequency (recovered
        # from row 1, whose angle is exactly freq)
        f1 = np.arctan2(s[1].astype(np.float64), c[1].astype(np.float64))
        assert np.all(np.abs(f1 - freq64) <= 4e-7 * freq64)
        ang = (np.arange(32768, dtype=np.float32)[:, None] * freq[None, :]).astype(np.float32).astype(np.float64)
        for got, want in ((c, np.cos(ang)), (s, np.sin(ang))):
            ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
            assert np.all(np.abs(got - want) <= ulp * 1.01 + 1e-30)
    cd, _ = orc.rope_lut_lfm2(32768, 64, 1e6)
    cf, _ = orc.rope_table_lfm2(32768, 64, 1e6)
    assert np.abs(cd[:1024] - cf[:1024]).max() < 1e-4 and np.abs(cd - cf).max() > 5e-4


def test_rope_table_lfm2_matches_reference(orc, ref):
    """Bit for bit against the tables the reference's own state initialisers
    build (lfm2_batch_state_init and lfm2_state_init, compiled from source)."""
    for hd, base in ((64, 1e6), (64, 1e4), (128, 1e6), (64, 0.0)):
        mine = orc.rope_table_lfm2(32768 if hd == 64 else 4096, hd, base)
        for which in (0, 1):
            theirs = ref.rope_table_lfm2(32768 if hd == 64 else 4096, hd, base, which=which)
            assert all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(mine, theirs))


def test_rope_table_lfm2_host_builder(orc):
    """lfm_attn_rope_table_lfm2 (the product's host C11 builder, no device
    needed) equals the oracle's table bit for bit."""
    import laii_amd as la
    for hd, base in ((64, 1e6), (128, 1e4)):
        mine = la.rope_table_lfm2(32768, hd, base)
        want = orc.rope_table_lfm2(32768, hd, base)
        assert all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(mine, want))


@pytest.mark.parametrize("hd", [64, 128, 48, 40, 16, 8])
def test_qk_norm_rope_table_matches_reference(orc, ref, hd):
    """orc_qk_norm_rope_table bit for bit against lfm2_qk_norm_and_rope_table
    and lfm2_qk_norm_and_rope (compiled from source) at the positions the
    production stacks reach (0 .. 32767), with and without norm weights, on
    inputs spanning six orders of magnitude; head dims with a scalar tail in
    the norm (40) and in the rotation (48, 40, 16, 8) included."""
    rng = np.random.default_rng(40 + hd)
    c, s = orc.rope_table_lfm2(32768, hd, 1e6)
    for pos in (0, 1, 1023, 8191, 32767):
        for norm in (True, False):
            x = (rng.standard_normal(8 * hd) * rng.choice([1e-3, 1.0, 40.0], 8 * hd)).astype(np.float32)
            w = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32) if norm else None
            mine = orc.qk_norm_rope(x, 8, hd, w, 1e-5, c[pos], s[pos], table=True)
            for which in (0, 1):
                theirs = ref.qk_norm_rope_table(x, 8, hd, w, 1e-5, c, s, pos, which=which)
                assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32)), (pos, norm, which)
            k16 = orc.qk_norm_rope(x, 8, hd, w, 1e-5, c[pos], s[pos], store_f16=True, table=True)
            assert np.array_equal(k16, ref.store_f16(mine))
            # float64 closed form with the table's own cos / sin
            want = _norm_rope_f64(x, 8, hd, w, 1e-5, c[pos], s[pos])
            assert np.abs(mine - want).max() <= 5e-6 * max(1.0, np.abs(want).max())


def test_qk_norm_rope_table_order_is_pinned(orc, ref):
    """The two LFM2 prologues add the squares in different orders; on these
    inputs the fast kernels' order (a plausible mix-up) is not bit-identical
    to lfm2_rmsnorm's, so the bit-exact check above tells them apart -- and
    so does one with the table swapped for the double-angle one."""
    rng = np.random.default_rng(11)
    c, s = orc.rope_table_lfm2(32768, 64, 1e6)
    cd, sd = orc.rope_lut_lfm2(32768, 64, 1e6)
    d_order = d_table = 0
    for _ in range(20):
        x = (rng.standard_normal(16 * 64) * 3).astype(np.float32)
        w = (1 + 0.05 * rng.standard_normal(64)).astype(np.float32)
        theirs = ref.qk_norm_rope_table(x, 16, 64, w, 1e-5, c, s, 32767)
        other_order = orc.qk_norm_rope(x, 16, 64, w, 1e-5, c[32767], s[32767])
        other_table = orc.qk_norm_rope(x, 16, 64, w, 1e-5, cd[32767], sd[32767], table=True)
        d_order += int(np.count_nonzero(other_order.view(np.uint32) != theirs.view(np.uint32)))
        d_table += int(np.count_nonzero(other_table.view(np.uint32) != theirs.view(np.uint32)))
    assert d_order > 0 and d_table > 0


# ---- A1/A2/A3/A7 attention ----------------------------------------------------------------------

def _brute(q, kf, vf, nq, nkv, hd, t0, t1, scale, gate=None, head_map=None):
    kv_mul = nq // nkv
    out = []
    for h in range(nq):
        kvh = head_map(h) if head_map else h // kv_mul
        o = softmax_attention_f64(q[h * hd:(h + 1) * hd], kf[t0:t1 + 1, kvh], vf[t0:t1 + 1, kvh], scale)
        out.append(o * (1.0 if gate is None else gate[h]))
    return np.concatenate(out)


def test_a1_closed_form(orc):
    rng = np.random.default_rng(5)
    nq, nkv, hd = 32, 8, 64
    k16 = f16(rng.standard_normal((600, nkv, hd)) * 0.5)
    v16 = f16(rng.standard_normal((600, nkv, hd)) * 0.5)
    kf, vf = f16_to_f32(k16), f16_to_f32(v16)
    for pos in (0, 1, 63, 599):
        q = rng.standard_normal(nq * hd).astype(np.float32)
        got = orc.online_gqa_f16(q, k16, v16, nq, 4, nkv * hd, pos)
        want = _brute(q, kf, vf, nq, nkv, hd, 0, pos, 0.125)
        assert np.abs(got - want).max() < 2e-6, pos


def test_a1_reference_golden(orc, gold):
    got = orc.online_gqa_f16(gold["a1_q"], gold["a1_k16"], gold["a1_v16"], 16, 4, 256, 37)
    assert np.abs(got - gold["a1_out"]).max() < 1e-6


def test_a2_branches(orc, gold):
    """FP32 two-pass branch vs the reference's golden output, and the
    tests/test_optimizations.c:324-421 single-head FP16 case (gate 5e-3)."""
    i = np.arange(128 * 256, dtype=np.float32)
    k = np.sin(i * np.float32(0.01)).astype(np.float32)
    v = np.cos(i * np.float32(0.02)).astype(np.float32)
    got = orc.gqa_heads(gold["a1_q"], 16, 4, 64, 256, 37, k32=k, v32=v)
    assert np.abs(got - gold["a2_f32_out"]).max() < 1e-6
    q1, k1, v1 = gold["a2_one_q"], gold["a2_one_k"], gold["a2_one_v"]
    got1 = orc.gqa_heads(q1, 1, 1, 64, 64, 31, k16=f16(k1), v16=f16(v1))
    assert np.abs(got1 - gold["a2_one_out"]).max() < 1e-6
    exact = softmax_attention_f64(q1, k1, v1, 0.125)
    assert np.abs(got1 - exact).max() < 5e-3


def test_a2_head_dim_quirk(orc):
    """tools/lfm2_threadpool.c:783: with head_dim > 64 the fp16 branch writes
    only 64 dims (the rest of the output keeps its previous contents)."""
    rng = np.random.default_rng(6)
    nq, nkv, hd = 4, 2, 128
    k16 = f16(rng.standard_normal((10, nkv, hd)))
    v16 = f16(rng.standard_normal((10, nkv, hd)))
    q = rng.standard_normal(nq * hd).astype(np.float32)
    init = np.full(nq * hd, -3.0, np.float32)
    got = orc.gqa_heads(q, nq, 2, hd, nkv * hd, 9, k16=k16, v16=v16, out=init).reshape(nq, hd)
    assert np.all(got[:, 64:] == -3.0)
    want = _brute(q, f16_to_f32(k16), f16_to_f32(v16), nq, nkv, hd, 0, 9, 1 / np.sqrt(np.float32(hd)))
    assert np.abs(got[:, :64] - want.reshape(nq, hd)[:, :64]).max() < 2e-6


def test_a3_ring_wrap_golden(orc, gold):
    """tests/test_lfm3.c:170-251 through 42 positions: golden outputs of the
    reference and the exact two-pass SWA softmax times the gate (1e-4)."""
    gate = gold["a3_gate"]
    nq, nkv, hd, win, cap = 8, 2, 128, 16, 24
    lin_k = np.zeros((42, nkv, hd), np.float32)
    lin_v = np.zeros((42, nkv, hd), np.float32)
    for p in range(42):
        kr, vr, q = gold["a3_k"][p], gold["a3_v"][p], gold["a3_q"][p]
        lin_k[p] = f16_to_f32(kr[p % cap]).reshape(nkv, hd)
        lin_v[p] = f16_to_f32(vr[p % cap]).reshape(nkv, hd)
        got = orc.lfm3_online_gqa_f16(q, gate, kr, vr, 1, p, win, cap, nq, nkv, hd)
        assert np.abs(got - gold["a3_out"][p]).max() < 1e-6
        t0 = max(0, p + 1 - win)
        want = _brute(q, lin_k, lin_v, nq, nkv, hd, t0, p, 1 / np.sqrt(np.float32(hd)), gate)
        assert np.abs(got - want).max() < 1e-5


def test_a3_rows_and_gate_absent(orc):
    rng = np.random.default_rng(8)
    nq, nkv, hd, win, cap = 16, 4, 128, 256, 264
    k16 = f16(rng.standard_normal((cap, nkv, hd)) * 0.5)
    v16 = f16(rng.standard_normal((cap, nkv, hd)) * 0.5)
    B, pos_0 = 4, 1000
    q = rng.standard_normal(B * nq * hd).astype(np.float32)
    got = orc.lfm3_online_gqa_f16(q, None, k16, v16, B, pos_0, win, cap, nq, nkv, hd)
    kf, vf = f16_to_f32(k16), f16_to_f32(v16)
    for b in range(B):
        p = pos_0 + b
        idx = [t % cap for t in range(p + 1 - win, p + 1)]
        want = _brute(q[b * nq * hd:(b + 1) * nq * hd], kf[idx], vf[idx], nq, nkv, hd, 0, win - 1,
                      1 / np.sqrt(np.float32(hd)))
        assert np.abs(got[b * nq * hd:(b + 1) * nq * hd] - want).max() < 2e-6


def test_causal_rows_closed_form(orc):
    rng = np.random.default_rng(9)
    nq, nkv, hd, n_rows, pos_0 = 32, 8, 64, 8, 300
    k16 = f16(rng.standard_normal((pos_0 + n_rows, nkv, hd)) * 0.5)
    v16 = f16(rng.standard_normal((pos_0 + n_rows, nkv, hd)) * 0.5)
    q = rng.standard_normal((n_rows, nq * hd)).astype(np.float32)
    got = orc.causal_rows_f16(q, k16, v16, n_rows, pos_0, nq, nkv, hd).reshape(n_rows, -1)
    kf, vf = f16_to_f32(k16), f16_to_f32(v16)
    for r in range(n_rows):
        want = _brute(q[r], kf, vf, nq, nkv, hd, 0, pos_0 + r, 0.125)
        assert np.abs(got[r] - want).max() < 2e-6


def test_decode_batch_mt_equals_single(orc):
    rng = np.random.default_rng(10)
    ks = [f16(rng.standard_normal((n, 8, 64)) * 0.5) for n in (100, 257, 31)]
    vs = [f16(rng.standard_normal((n, 8, 64)) * 0.5) for n in (100, 257, 31)]
    pos = np.array([99, 256, 30], np.uint32)
    q = rng.standard_normal((3, 32 * 64)).astype(np.float32)
    got = orc.decode_batch_mt(q, ks, vs, pos, 32, 8, 64, 4).reshape(3, -1)
    for s in range(3):
        assert np.array_equal(got[s], orc.online_gqa_f16(q[s], ks[s], vs[s], 32, 4, 512, int(pos[s])))


def test_reference_batch_dispatches_agree(orc, ref):
    """The two CPU-baseline dispatches of the reference's decode worker (per
    sequence through its pool, and every (sequence, head group) item across
    threads) give bit-identical rows, equal to the oracle's batch."""
    rng = np.random.default_rng(12)
    ks = [f16(rng.standard_normal((n, 8, 64)) * 0.5) for n in (100, 257, 31, 64)]
    vs = [f16(rng.standard_normal((n, 8, 64)) * 0.5) for n in (100, 257, 31, 64)]
    pos = np.array([99, 256, 30, 63], np.uint32)
    q = rng.standard_normal((4, 32 * 64)).astype(np.float32)
    _, _, per_seq = ref.time_decode_batch(q, ks, vs, pos, 32, 8, 3, 1)
    _, fair = ref.time_decode_batch_fair(q, ks, vs, pos, 32, 8, 3, 2)
    assert np.array_equal(per_seq, fair)
    want = orc.decode_batch_mt(q, ks, vs, pos, 32, 8, 64, 2)
    assert np.abs(fair - want.reshape(-1)).max() < 1e-6


def test_attention_matches_reference_build(orc, ref):
    rng = np.random.default_rng(11)
    nq, nkv, hd, pos = 32, 8, 64, 999
    k16 = f16(rng.standard_normal((1000, nkv, hd)) * 0.5)
    v16 = f16(rng.standard_normal((1000, nkv, hd)) * 0.5)
    q = rng.standard_normal(nq * hd).astype(np.float32)
    assert np.abs(orc.online_gqa_f16(q, k16, v16, nq, 4, 512, pos) -
                  ref.online_gqa_f16(q, k16, v16, nq, 4, 512, pos)).max() < 1e-6
    assert np.abs(orc.gqa_heads(q, nq, 4, hd, 512, pos, k16=k16, v16=v16) -
                  ref.gqa_heads(q, nq, 4, hd, 512, 1000, pos, k16=k16, v16=v16)).max() < 1e-6
    nq, nkv, hd, cap = 16, 4, 128, 264
    k16 = f16(rng.standard_normal((cap, nkv, hd)) * 0.5)
    v16 = f16(rng.standard_normal((cap, nkv, hd)) * 0.5)
    q = rng.standard_normal(3 * nq * hd).astype(np.float32)
    g = rng.random(3 * nq).astype(np.float32)
    assert np.abs(orc.lfm3_online_gqa_f16(q, g, k16, v16, 3, 1000, 256, cap, nq, nkv, hd) -
                  ref.lfm3_dispatch(q, g, k16, v16, 3, 1000, 256, cap, nq, nkv, hd)).max() < 1e-6


# ---- A6: Gen-1 FP32 step against the reference's PyTorch fixture -------------------------------

def test_gen1_fixture(orc):
    """tests/fixtures_attention.bin (tools/generate_reference_tensors.py:77-164,
    gate 1e-4 in tests/test_attention.c:105): projections and wo are done here
    in float64; norm, RoPE, FP32 append and two-pass attention by the oracle."""
    raw = open(os.path.join(GOLDEN, "fixtures_attention.bin"), "rb").read()
    D, nq, nkv, hd, pos, _ = struct.unpack("6I", raw[:24])
    f = np.frombuffer(raw[24:], np.float32)
    o = 0

    def take(n, shape):
        nonlocal o
        a = f[o:o + n].reshape(shape)
        o += n
        return a

    x = take(D, (D,))
    wq, wk, wv = take(nq * hd * D, (nq * hd, D)), take(nkv * hd * D, (nkv * hd, D)), take(nkv * hd * D, (nkv * hd, D))
    qn, kn = take(hd, (hd,)), take(hd, (hd,))
    wo = take(D * D, (D, D))
    kh, vh = take(pos * nkv * hd, (pos, nkv * hd)), take(pos * nkv * hd, (pos, nkv * hd))
    expected = take(D, (D,))
    assert o == f.size
    q = (wq.astype(np.float64) @ x).astype(np.float32)
    k = (wk.astype(np.float64) @ x).astype(np.float32)
    v = (wv.astype(np.float64) @ x).astype(np.float32)
    kc = np.zeros((pos + 10, nkv * hd), np.float32)
    vc = np.zeros((pos + 10, nkv * hd), np.float32)
    kc[:pos], vc[:pos] = kh, vh
    attn = orc.gen1_gqa_attend(q, k, v, qn, kn, kc, vc, pos, nq, nkv, hd, 1e-5, 1e6)
    out = wo.astype(np.float64) @ attn
    assert np.abs(out - expected).max() < 1e-4


def _gen1_one_hot_case(rng, nq, nkv, hd, pos):
    """Inputs for lfm_gqa_step whose projections and wo are exact: x is the
    one-hot e_0 (each projected value is one weight) and wo the identity, so
    the step's output is its attention output bit for bit."""
    D = nq * hd
    x = np.zeros(D, np.float32)
    x[0] = 1.0
    wq = rng.standard_normal((nq * hd, D)).astype(np.float32)
    wk = rng.standard_normal((nkv * hd, D)).astype(np.float32)
    wv = rng.standard_normal((nkv * hd, D)).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kc = rng.standard_normal((pos + 3, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((pos + 3, nkv * hd)).astype(np.float32)
    return x, wq, wk, wv, np.eye(D, dtype=np.float32), qn, kn, kc, vc


@pytest.mark.parametrize("nq,nkv,hd,pos", [(4, 2, 16, 5), (32, 8, 64, 300), (16, 4, 128, 77), (8, 8, 40, 0),
                                            (12, 4, 96, 1000)])
def test_gen1_bit_exact_vs_reference_step(orc, ref_gen1, nq, nkv, hd, pos):
    """The oracle's Gen-1 step against the reference's own lfm_gqa_step
    (src/lfm_forward.c:162-248, compiled from its sources): attention output
    and the appended cache rows bit for bit -- the AVX2 sums of squares and
    dot products in their column order, powf/cosf/sinf angles, two-pass
    softmax."""
    rng = np.random.default_rng(pos + hd)
    x, wq, wk, wv, wo, qn, kn, kc, vc = _gen1_one_hot_case(rng, nq, nkv, hd, pos)
    kc2, vc2 = kc.copy(), vc.copy()
    out = ref_gen1.gqa_step(x, wq, wk, wv, wo, qn, kn, kc, vc, pos, nq, nkv, hd, 1e-5, 1e6)
    att = orc.gen1_gqa_attend(wq[:, 0].copy(), wk[:, 0].copy(), wv[:, 0].copy(), qn, kn, kc2, vc2, pos, nq, nkv,
                              hd, 1e-5, 1e6)
    assert np.array_equal(out.view(np.uint32), att.view(np.uint32))
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)


# ---- planted mistakes: the checks above are sensitive ------------------------------------------

def test_planted_mistakes_are_caught(orc):
    rng = np.random.default_rng(12)
    nq, nkv, hd, pos = 32, 8, 64, 200
    k16 = f16(rng.standard_normal((pos + 1, nkv, hd)) * 0.5)
    v16 = f16(rng.standard_normal((pos + 1, nkv, hd)) * 0.5)
    kf, vf = f16_to_f32(k16), f16_to_f32(v16)
    q = rng.standard_normal(nq * hd).astype(np.float32)
    got = orc.online_gqa_f16(q, k16, v16, nq, 4, nkv * hd, pos)
    tol = 2e-6
    assert np.abs(got - _brute(q, kf, vf, nq, nkv, hd, 0, pos, 0.125)).max() < tol
    mutants = {
        "kv head h % n_kv instead of h / kv_mul": _brute(q, kf, vf, nq, nkv, hd, 0, pos, 0.125,
                                                         head_map=lambda h: h % nkv),
        "K and V swapped": _brute(q, vf, kf, nq, nkv, hd, 0, pos, 0.125),
        "last key dropped": _brute(q, kf, vf, nq, nkv, hd, 0, pos - 1, 0.125),
        "first key dropped": _brute(q, kf, vf, nq, nkv, hd, 1, pos, 0.125),
        "scale missing": _brute(q, kf, vf, nq, nkv, hd, 0, pos, 1.0),
        "K transposed within the head": _brute(q, kf[:, :, ::-1], vf, nq, nkv, hd, 0, pos, 0.125),
    }
    for name, wrong in mutants.items():
        assert np.abs(got - wrong).max() > 100 * tol, name
    # ring: reading seg2 from seg1_slot instead of slot 0 is caught by the slot walk
    walk = orc.lfm3_slots(1000, 256, 264)
    wrong_walk = [217 + t for t in range(47)] + [217 + t for t in range(209)]
    assert list(walk) != wrong_walk
