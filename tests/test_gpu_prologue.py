"""GPU parity of the QK-RMSNorm + RoPE + RNE fp16 store prologue."""
import numpy as np
import pytest

from helpers import f16, parity

pytestmark = pytest.mark.gpu


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def test_store_fp32_to_fp16_bit_exact(gpu):
    """A8: RNE conversion, bit-exact incl. ties, subnormals, overflow and signed zero."""
    la = gpu
    rng = np.random.default_rng(0)
    hv = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((hv[:-1] + hv[1:]) / 2).astype(np.float32)
    x = np.concatenate([rng.standard_normal(1 << 16).astype(np.float32) * s
                        for s in (1e-7, 1e-5, 1e-2, 1.0, 1e3)] +
                       [mids, -mids, np.array([65504, 65519.99, 65520, 1e9, -1e9, 0.0, -0.0,
                                               2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -25],
                                              np.float32)]).astype(np.float32)
    dst = la.DeviceArray(x.size, np.uint16)
    la.store_fp32_to_fp16(dst, dev(la, x), x.size)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = dst.numpy()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (x[bad[:5]], got[bad[:5]], want[bad[:5]])


@pytest.mark.parametrize("hd,base,rope_dim,partial", [(64, 1e6, 64, False), (128, 1e4, 128, False),
                                                       (128, 1e6, 128, True)])
def test_qk_norm_rope(gpu, orc, hd, base, rope_dim, partial):
    """A4/A5 for Q (fp32 in place) and K (RNE fp16 store), bit for bit: the
    oracle follows the reference's AVX2 kernels exactly at d64 and d128."""
    la = gpu
    rng = np.random.default_rng(hd)
    n_heads, max_seq, pos, eps = 16, 2048, 1337, 1e-5
    rf = np.array([1.0] * (hd // 4) + [1e30] * (hd // 4), np.float32) if partial else None
    if hd == 64:
        cos, sin = la.rope_lut_lfm2(max_seq, hd, base)
    else:
        cos, sin = la.rope_lut_lfm3(max_seq, hd, rope_dim, base, rf)
    x = rng.standard_normal(n_heads * hd, dtype=np.float32) * np.float32(3.0)
    w = (np.float32(1.0) + np.float32(0.05) * rng.standard_normal(hd, dtype=np.float32)).astype(np.float32)
    cd, sd, wd = dev(la, cos), dev(la, sin), dev(la, w)
    xq = dev(la, x)
    la.qk_norm_rope(xq, None, n_heads, hd, wd, eps, cd, sd, pos)
    want_q = orc.qk_norm_rope(x, n_heads, hd, w, eps, cos[pos], sin[pos])
    # the oracle is bit-identical to the reference's AVX2 kernels at d64 / d128
    assert np.array_equal(xq.numpy().view(np.uint32), want_q.view(np.uint32)), f"Q norm+rope hd={hd}"
    k16 = la.DeviceArray.zeros(n_heads * hd, np.uint16)
    xk = dev(la, x)
    la.qk_norm_rope(xk, k16, n_heads, hd, wd, eps, cd, sd, pos)
    assert np.array_equal(xk.numpy(), x), "fp16-store mode must leave the source untouched"
    want_k = orc.qk_norm_rope(x, n_heads, hd, w, eps, cos[pos], sin[pos], store_f16=True)
    assert np.array_equal(k16.numpy(), want_k), f"K fp16 store hd={hd}"
    if partial:  # dims of identity pairs are the normalised input, unrotated
        keep = np.r_[hd // 4:hd // 2, 3 * hd // 4:hd]
        normed = orc.qk_norm_rope(x, n_heads, hd, w, eps, np.ones(hd // 2, np.float32),
                                  np.zeros(hd // 2, np.float32))
        got = xq.numpy().reshape(n_heads, hd)[:, keep]
        assert np.allclose(got, normed.reshape(n_heads, hd)[:, keep], rtol=0, atol=2e-6)


def test_qkv_prologue_batched(gpu, orc):
    """Batched prologue: many sequences x rows, ring slots, V store bit-exact."""
    la = gpu
    rng = np.random.default_rng(9)
    n_seq, n_rows, nq, nkv, hd, win, cap, eps = 5, 3, 16, 4, 128, 256, 264, 1e-5
    cos, sin = la.rope_lut_lfm3(4096, hd, hd, 1e4, None)
    pos0 = np.array([0, 255, 262, 1000, 3000], np.uint32)
    q = rng.standard_normal((n_seq, n_rows, nq, hd), dtype=np.float32)
    k = rng.standard_normal((n_seq, n_rows, nkv, hd), dtype=np.float32)
    v = rng.standard_normal((n_seq, n_rows, nkv, hd), dtype=np.float32)
    qw = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
    caches_k = [la.DeviceArray.zeros((cap, nkv, hd), np.uint16) for _ in range(n_seq)]
    caches_v = [la.DeviceArray.zeros((cap, nkv, hd), np.uint16) for _ in range(n_seq)]
    qd = dev(la, q)
    la.qkv_prologue(qd, dev(la, k), dev(la, v), la.pointer_table(caches_k),
                    la.pointer_table(caches_v), dev(la, pos0), n_seq, n_rows, nq, nkv, hd,
                    dev(la, qw), dev(la, kw), eps, dev(la, cos), dev(la, sin), win, cap)
    gq = qd.numpy()
    for s in range(n_seq):
        ks, vs = caches_k[s].numpy(), caches_v[s].numpy()
        for r in range(n_rows):
            p = int(pos0[s]) + r
            slot = p % cap
            assert la.slot_of(p, win, cap) == slot
            wq = orc.qk_norm_rope(q[s, r], nq, hd, qw, eps, cos[p], sin[p])
            assert np.array_equal(gq[s, r].reshape(-1).view(np.uint32), wq.view(np.uint32)), f"q s={s} r={r}"
            wk = orc.qk_norm_rope(k[s, r], nkv, hd, kw, eps, cos[p], sin[p], store_f16=True)
            assert np.array_equal(ks[slot].reshape(-1), wk), f"k s={s} r={r}"
            assert np.array_equal(vs[slot].reshape(-1), f16(v[s, r]).reshape(-1))
