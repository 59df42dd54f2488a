"""Attention-sink eviction: pins of the oracle restatement
(orc_kv_shift_sinks_lfm2 / _lfm3) against the reference's own shift kernels
compiled from source (bit-exact), against the rotation algebra
R(-d) R(p) = R(p - d), and on the no-op cases
(tools/lfm2_runtime_features.c:744-833, 1055-1163; tests mirrored from
tests/test_runtime_features.c:356-494 and tests/test_lfm3.c:515-524)."""
import numpy as np
import pytest

from helpers import f16_to_f32

RF_PARTIAL = np.array([1.0] * 32 + [1e30] * 32, np.float32)


def lut2(orc, rows, hd=64, base=1e6):
    c, s = orc.rope_lut_lfm2(rows, hd, base)
    return np.ascontiguousarray(c), np.ascontiguousarray(s)


def lut3(orc, rows, hd, base, rope_freqs=None):
    c, s = orc.rope_lut_lfm3(rows, hd, hd, base, rope_freqs)
    return np.ascontiguousarray(c), np.ascontiguousarray(s)


def rand_cache(rng, rows, kv_dim, scale=1.5):
    return (rng.standard_normal((rows, kv_dim)) * scale).astype(np.float16).view(np.uint16)


def copies(caches):
    return [None if c is None else c.copy() for c in caches]


@pytest.mark.parametrize("pos,n_sink,n_discard", [
    (290, 16, 50),    # overlapping move (n_keep 224 > n_discard)
    (290, 16, 200),   # disjoint move
    (300, 0, 1),      # no sinks, one-row shift
    (200, 16, 64),    # tests/test_runtime_features.c:454-466
    (100, 40, 60),    # pos == n_sink + n_discard: no-op
    (50, 40, 60),     # below: no-op
    (290, 16, 0),     # n_discard 0: no-op
])
def test_lfm2_shift_matches_reference(orc, ref, pos, n_sink, n_discard):
    rng = np.random.default_rng(pos + 7 * n_discard)
    rows, hd = 300, 64
    nkv = [0, 8, 2]  # ShortConv layer, 8-head and 2-head GQA layers
    K = [None] + [rand_cache(rng, rows, n * hd) for n in nkv[1:]]
    V = [None] + [rand_cache(rng, rows, n * hd, 1.0) for n in nkv[1:]]
    Kr, Vr = copies(K), copies(V)
    lut = lut2(orc, rows)
    p_o = orc.kv_shift_sinks_lfm2(K, V, nkv, hd, lut, pos, n_sink, n_discard)
    p_r = ref.kv_shift_sinks_lfm2(Kr, Vr, nkv, hd, lut, pos, n_sink, n_discard)
    assert p_o == p_r
    if n_discard == 0 or pos <= n_sink + n_discard:
        assert p_o == pos
    else:
        assert p_o == pos - n_discard
    for a, b in zip(K[1:] + V[1:], Kr[1:] + Vr[1:]):
        assert np.array_equal(a, b)


def test_lfm2_head_dim_other_than_64_is_noop(orc, ref):
    rng = np.random.default_rng(3)
    K = [rand_cache(rng, 64, 4 * 128)]
    V = [rand_cache(rng, 64, 4 * 128)]
    K0, V0 = copies(K), copies(V)
    lut = lut2(orc, 64, 128)
    assert orc.kv_shift_sinks_lfm2(K, V, [4], 128, lut, 60, 4, 10) == 60
    assert ref.kv_shift_sinks_lfm2(copies(K0), copies(V0), [4], 128, lut, 60, 4, 10) == 60
    assert np.array_equal(K[0], K0[0]) and np.array_equal(V[0], V0[0])


@pytest.mark.parametrize("cap,win,pos,n_sink,n_discard", [
    (264, 256, 600, 64, 300),   # engine geometry (w + 8), window fully past the sinks
    (256, 256, 1000, 64, 500),  # cap == window (BASELINE cfg 5 ring)
    (24, 16, 60, 4, 10),        # tests/test_lfm3.c:515-524 shape, window reaches the sinks
    (24, 16, 30, 8, 12),        # new_pos 18: window covers sink rows
    (40, 16, 39, 2, 30),        # small new_pos (11 < window)
])
def test_lfm3_shift_matches_reference(orc, ref, cap, win, pos, n_sink, n_discard):
    rng = np.random.default_rng(cap + pos)
    hd, nkv = 128, 4
    rows_full = pos + 8
    kinds = [1, 2, 0, 2]
    K = [rand_cache(rng, rows_full, nkv * hd), rand_cache(rng, cap, nkv * hd), None,
         rand_cache(rng, cap, nkv * hd)]
    V = [rand_cache(rng, rows_full, nkv * hd), rand_cache(rng, cap, nkv * hd), None,
         rand_cache(rng, cap, nkv * hd)]
    Kr, Vr = copies(K), copies(V)
    lf = lut3(orc, rows_full, hd, 1e6, RF_PARTIAL)
    lw = lut3(orc, rows_full, hd, 1e4)
    args = ([nkv, nkv, 0, nkv], kinds, hd, lf, lw, win, cap, pos, n_sink, n_discard)
    p_o = orc.kv_shift_sinks_lfm3(K, V, *args)
    p_r = ref.kv_shift_sinks_lfm3(Kr, Vr, *args)
    assert p_o == p_r == pos - n_discard
    for a, b in zip(K, Kr):
        assert (a is None and b is None) or np.array_equal(a, b)
    for a, b in zip(V, Vr):
        assert (a is None and b is None) or np.array_equal(a, b)


def test_lfm3_noop_cases(orc, ref):
    rng = np.random.default_rng(5)
    hd, nkv = 128, 4
    K = [rand_cache(rng, 64, nkv * hd)]
    V = [rand_cache(rng, 64, nkv * hd)]
    lf = lut3(orc, 64, hd, 1e6)
    for pos, n_sink, n_discard in ((40, 8, 32), (60, 8, 0), (60, 8, 64)):  # last: n_discard >= rows
        K0, V0 = copies(K), copies(V)
        for impl in (orc, ref):
            Kc, Vc = copies(K0), copies(V0)
            assert impl.kv_shift_sinks_lfm3(Kc, Vc, [nkv], [1], hd, lf, lf, 16, 24, pos, n_sink,
                                            n_discard) == pos
            assert np.array_equal(Kc[0], K0[0]) and np.array_equal(Vc[0], V0[0])


def roped_keys(orc, k_raw, n_heads, hd, lut, positions):
    """Keys RoPE-rotated at the given positions (no norm), stored RNE fp16."""
    c, s = lut
    out = np.empty((len(positions), n_heads * hd), np.uint16)
    for i, p in enumerate(positions):
        out[i] = orc.qk_norm_rope(k_raw[i].copy(), n_heads, hd, None, 1e-5, c[p], s[p],
                                  store_f16=True)
    return out


@pytest.mark.parametrize("kind", ["lfm2", "lfm3_full_partial", "lfm3_swa"])
def test_counter_rotation_composes(orc, kind):
    """A key roped at position p and shifted by n_discard equals the same key
    roped at p - n_discard, to fp16 round-trip accuracy -- the reference's own
    acceptance test (tests/test_runtime_features.c:356-423, bound 1.5e-3)."""
    rng = np.random.default_rng(11)
    n_sink, n_discard, pos = 8, 40, 120
    if kind == "lfm2":
        hd, nkv, lut = 64, 8, lut2(orc, 256)
    elif kind == "lfm3_full_partial":
        hd, nkv, lut = 128, 4, lut3(orc, 256, 128, 1e6, RF_PARTIAL)
    else:
        hd, nkv, lut = 128, 4, lut3(orc, 256, 128, 1e4)
    # the reference test's inputs: cos(0.023 i) * 1.5 (|k| <= 1.5, so one fp16
    # ulp is at most 2^-10 and two roundings stay under its 1.5e-3 bound)
    k_raw = (np.cos(np.arange(pos * nkv * hd, dtype=np.float32) * np.float32(0.023))
             * np.float32(1.5)).reshape(pos, nkv * hd)
    K = roped_keys(orc, k_raw, nkv, hd, lut, list(range(pos)))
    V = rand_cache(rng, pos, nkv * hd)
    kept = list(range(n_sink + n_discard, pos))
    want = roped_keys(orc, k_raw[kept], nkv, hd, lut, [t - n_discard for t in kept])
    if kind == "lfm2":
        new = orc.kv_shift_sinks_lfm2([K], [V], [nkv], hd, lut, pos, n_sink, n_discard)
        got = K[n_sink:new]
    elif kind == "lfm3_full_partial":
        new = orc.kv_shift_sinks_lfm3([K], [V], [nkv], [1], hd, lut, lut, 16, 24, pos, n_sink,
                                      n_discard)
        got = K[n_sink:new]
    else:
        cap, win = 40, 32
        ring = np.zeros((cap, nkv * hd), np.uint16)
        vring = np.zeros_like(ring)
        for t in range(pos - cap, pos):  # the ring holds the last cap positions
            ring[t % cap] = K[t]
            vring[t % cap] = V[t]
        new = orc.kv_shift_sinks_lfm3([ring], [vring], [nkv], [2], hd, lut, lut, win, cap, pos,
                                      n_sink, n_discard)
        got = np.stack([ring[t % cap] for t in range(new - win, new)])
        want = want[-win:]
        assert np.array_equal(np.stack([vring[t % cap] for t in range(new - win, new)]),
                              V[new - win + n_discard:pos])
    assert new == pos - n_discard
    err = np.abs(f16_to_f32(got) - f16_to_f32(want)).max()
    assert err < 1.5e-3, err
    if kind == "lfm3_full_partial":
        # unrotated dims (32..63, 96..127) move bit-exactly
        idx = np.concatenate([np.arange(32, 64), np.arange(96, 128)])
        g = got.reshape(len(got), nkv, hd)[:, :, idx]
        w = K.reshape(pos, nkv, hd)[n_sink:new]  # already shifted in place
        assert np.array_equal(g, w[:, :, idx])


def test_planted_sign_error_breaks_composition(orc):
    """A counter-rotation with the wrong direction (a plausible mistake) fails
    the composition check: rotating by +n_discard instead lands 2*n_discard
    away from the target position."""
    rng = np.random.default_rng(2)
    hd, nkv, n_discard = 64, 2, 40
    lut = lut2(orc, 256)
    k_raw = rng.standard_normal((1, nkv * hd)).astype(np.float32)
    p = 100
    K = roped_keys(orc, k_raw, nkv, hd, lut, [p])
    want = roped_keys(orc, k_raw, nkv, hd, lut, [p - n_discard])
    wrong = roped_keys(orc, k_raw, nkv, hd, lut, [p + n_discard])
    assert np.abs(f16_to_f32(wrong) - f16_to_f32(want)).max() > 0.05
    # the oracle's direction is the right one
    cache = np.zeros((p + 1, nkv * hd), np.uint16)
    cache[p] = K[0]
    v = np.zeros_like(cache)
    orc.kv_shift_sinks_lfm2([cache], [v], [nkv], hd, lut, p + 1, 0, n_discard)
    got, w = f16_to_f32(cache[p - n_discard]), f16_to_f32(want[0])
    ulp = np.spacing(np.maximum(np.abs(got), np.abs(w)).astype(np.float16)).astype(np.float32)
    assert np.all(np.abs(got - w) <= 2 * ulp)  # two fp16 roundings
