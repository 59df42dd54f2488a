"""GPU parity of the causal MFMA prefill against the oracle's causal rows
(tools/lfm2_prefill_batch.c:1029-1092 semantics: row i at position pos_0 + i
attends keys [0, pos_0 + i])."""
import numpy as np
import pytest

from helpers import f16, f16_to_f32, parity, rand_kv

pytestmark = pytest.mark.gpu


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def run_prefill(la, rng, n_seq, n_tok, pos_0, nq, nkv, hd=64, scale_qkv=0.5):
    """fp32 Q (the reference's rows), fp16 K/V caches."""
    slots = pos_0 + n_tok
    q = rng.standard_normal((n_seq, n_tok, nq, hd), dtype=np.float32) * np.float32(scale_qkv)
    k16 = np.stack([rand_kv(rng, slots, nkv, hd, scale_qkv) for _ in range(n_seq)])
    v16 = np.stack([rand_kv(rng, slots, nkv, hd, scale_qkv) for _ in range(n_seq)])
    out = la.DeviceArray.zeros((n_seq, n_tok, nq, hd), np.float32)
    la.prefill_f16(dev(la, q), dev(la, k16), dev(la, v16), out, n_seq, n_tok, pos_0,
                   slots * nkv * hd, nq, nkv, hd)
    return q, k16, v16, out.numpy()


def oracle_rows(orc, q, k16, v16, s, rows, pos_0, nq, nkv, hd=64):
    """Oracle causal rows for the given row indices of sequence s (fp32 q)."""
    qf = np.asarray(q[s], dtype=np.float32)
    out = []
    for r in rows:
        out.append(orc.causal_rows_f16(qf[r], k16[s], v16[s], 1, pos_0 + r, nq, nkv, hd))
    return np.stack(out).reshape(len(rows), nq, hd)


@pytest.mark.parametrize("n_seq,n_tok,pos_0,nq,nkv", [
    (2, 512, 0, 32, 8),     # config 4 shape, reduced length
    (1, 200, 300, 32, 8),   # chunked prefill after an existing context
    (1, 100, 0, 32, 8),     # rows not a multiple of the query tile
    (1, 257, 5, 16, 8),     # kv_mul 2 (LFM2-350M-like heads)
    (1, 130, 0, 32, 4),     # kv_mul 8
    (1, 70, 0, 8, 8),       # kv_mul 1
])
def test_prefill_vs_oracle(gpu, orc, n_seq, n_tok, pos_0, nq, nkv):
    rng = np.random.default_rng(n_tok * 7 + pos_0 + nq)
    q, k16, v16, got = run_prefill(gpu, rng, n_seq, n_tok, pos_0, nq, nkv)
    for s in range(n_seq):
        want = oracle_rows(orc, q, k16, v16, s, range(n_tok), pos_0, nq, nkv)
        parity(got[s], want, what=f"prefill s={s} n={n_tok} pos0={pos_0} {nq}q/{nkv}kv")


def test_prefill_cfg4_full_size_sampled(gpu, orc):
    """BASELINE config 4 at full size (N 4096, B 4, 32q/8kv): sampled rows
    against the oracle, and every row's output is a convex combination of V
    rows (|o| <= max |v| per dim), the size-independent property."""
    rng = np.random.default_rng(4096)
    q, k16, v16, got = run_prefill(gpu, rng, 4, 4096, 0, 32, 8)
    for s in range(4):
        rows = [0, 1, 63, 64, 1000, 2047, 2048, 4095]
        want = oracle_rows(orc, q, k16, v16, s, rows, 0, 32, 8)
        parity(got[s][rows], want, what=f"prefill cfg4 s={s} sampled")
    vmax = np.abs(f16_to_f32(v16)).max()
    assert np.all(np.isfinite(got)) and np.abs(got).max() <= vmax + 1e-3
    # row 0 attends only key 0: its output is exactly V[0] of its KV head
    v0 = f16_to_f32(v16[:, 0])  # [s][kv][d]
    assert np.allclose(got[:, 0], np.repeat(v0, 4, axis=1), atol=1e-6)


def test_prefill_matches_decode_path(gpu):
    """The last prefill row equals the split-KV decode kernel at that position
    (two independent kernels, same cache)."""
    la = gpu
    rng = np.random.default_rng(77)
    n_tok, nq, nkv, hd = 1000, 32, 8, 64
    q, k16, v16, got = run_prefill(la, rng, 1, n_tok, 0, nq, nkv)
    out = la.DeviceArray.zeros(nq * hd, np.float32)
    qf = np.ascontiguousarray(q[0, n_tok - 1])
    la.online_gqa_f16(dev(la, qf), dev(la, k16[0]), dev(la, v16[0]), out, nq, 4, nkv * hd,
                      n_tok - 1, 0.125)
    parity(got[0, n_tok - 1].reshape(-1), out.numpy(), what="prefill last row vs decode")


def test_prefill_rejects_unsupported(gpu):
    la = gpu
    lib = la.load()
    a = la.DeviceArray.zeros(1 << 16, np.uint16)
    o = la.DeviceArray.zeros(1 << 16, np.float32)
    assert lib.lfm_hip_prefill_f16(o.ptr, a.ptr, a.ptr, o.ptr, 1, 8, 0, 0, 8, 2, 128, 0.088,
                                   None) == -3


@pytest.mark.parametrize("pattern", ["rising", "spike", "falling", "sunk"])
def test_prefill_lazy_max_raises(gpu, orc, pattern):
    """Score patterns that force the lazy running max to be raised after the
    first step (and in masked diagonal steps): keys whose scores climb by tens
    of log2 units along the sequence ("rising"), isolated huge scores
    ("spike"), a large first block followed by tiny ones ("falling"), and a
    first step whose scores all lie below -128 log2 units, where exp2(-m)
    overflows and must not scale the (zero) accumulators ("sunk").
    Against the oracle's causal rows."""
    la = gpu
    rng = np.random.default_rng({"rising": 1, "spike": 2, "falling": 3, "sunk": 4}[pattern])
    n_seq, n_tok, nq, nkv, hd = 1, 300, 16, 4, 64
    q = rng.standard_normal((n_seq, n_tok, nq, hd), dtype=np.float32)
    k = rng.standard_normal((n_seq, n_tok, nkv, hd), dtype=np.float32) * 0.5
    # a shared direction so that every query scores each key by its scale
    u = rng.standard_normal(hd).astype(np.float32)
    u /= np.linalg.norm(u)
    q += 3.0 * u
    t = np.arange(n_tok, dtype=np.float32)
    if pattern == "rising":
        amp = 0.25 * t          # scores grow ~ 0.125 * 3 * 0.25 t: +28 log2 units by the end
    elif pattern == "spike":
        amp = np.where(t % 97 == 40, 60.0, 0.0).astype(np.float32)
    elif pattern == "falling":
        amp = np.where(t < 64, 40.0, 0.0).astype(np.float32)
    else:
        amp = np.where(t < 32, -400.0, 0.0).astype(np.float32)
    k += amp[None, :, None, None] * u
    k16 = f16(k)
    v16 = f16(rng.standard_normal((n_seq, n_tok, nkv, hd), dtype=np.float32))
    out = la.DeviceArray.zeros((n_seq, n_tok, nq, hd), np.float32)
    la.prefill_f16(dev(la, q), dev(la, k16), dev(la, v16), out, n_seq, n_tok, 0,
                   n_tok * nkv * hd, nq, nkv, hd)
    got = out.numpy()
    assert np.all(np.isfinite(got))
    want = oracle_rows(orc, q, k16, v16, 0, range(n_tok), 0, nq, nkv)
    parity(got[0], want, what=f"prefill lazy max {pattern}")
