"""GPU parity of the head_dim-128 MFMA prefill (LFM3 full and sliding-window
layers, output gate; lfm_hip_lfm3_prefill_f16) against the oracle's batched
LFM3 attention (tools/lfm3_engine.c:1918-2055: the row at position p attends
keys [t_start(p), p], t_start from :862-873, scaled by sigmoid(gate) as at
:902-911)."""
import numpy as np
import pytest

from helpers import f16, f16_to_f32, parity, rand_kv

pytestmark = pytest.mark.gpu

HD = 128


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def t_start(p, window):
    return p + 1 - window if window and p + 1 > window else 0


def sigmoid(g):
    return (1.0 / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32)


def run(la, rng, n_seq, n_tok, pos_0, nq, nkv, window=0, kv_pos0=0, gate=True, q=None, k16=None, v16=None, hd=HD,
        gate_values=None):
    """fp32 Q rows, fp16 K/V buffers whose row r is position kv_pos0 + r
    (gate logits drawn unless gate_values are given)."""
    HD = hd
    rows = pos_0 + n_tok - kv_pos0
    if q is None:
        q = rng.standard_normal((n_seq, n_tok, nq, HD), dtype=np.float32) * np.float32(0.5)
    if k16 is None:
        k16 = np.stack([rand_kv(rng, rows, nkv, HD) for _ in range(n_seq)])
    if v16 is None:
        v16 = np.stack([rand_kv(rng, rows, nkv, HD) for _ in range(n_seq)])
    g = gate_values if gate_values is not None else (
        rng.standard_normal((n_seq, n_tok, nq)).astype(np.float32) if gate else None)
    out = la.DeviceArray.zeros((n_seq, n_tok, nq, HD), np.float32)
    la.lfm3_prefill_f16(dev(la, q), dev(la, k16), dev(la, v16), None if g is None else dev(la, g), True, out, n_seq,
                        n_tok, pos_0, kv_pos0, rows * nkv * HD, window, nq, nkv, HD)
    return q, k16, v16, g, out.numpy()


def oracle(orc, q, k16, v16, g, s, pos_0, kv_pos0, window, nq, nkv, rows=None):
    """The oracle on a cache of absolute positions: rows below kv_pos0 hold
    fp16 NaN, so reading one would poison the result."""
    n_tok, HD = q.shape[1], q.shape[-1]
    cap = max(pos_0 + n_tok, window)
    kf = np.full((cap, nkv, HD), 0x7E00, np.uint16)
    vf = np.full((cap, nkv, HD), 0x7E00, np.uint16)
    kf[kv_pos0:pos_0 + n_tok] = k16[s]
    vf[kv_pos0:pos_0 + n_tok] = v16[s]
    rows = range(n_tok) if rows is None else rows
    out = []
    for r in rows:
        gs = None if g is None else sigmoid(g[s, r])
        out.append(orc.lfm3_online_gqa_f16(q[s, r], gs, kf, vf, 1, pos_0 + r, window, cap, nq, nkv, HD))
    return np.stack(out).reshape(len(rows), nq, HD)


@pytest.mark.parametrize("n_seq,n_tok,pos_0,nq,nkv,gate", [
    (2, 300, 0, 16, 4, True),    # LFM3 heads, gated
    (1, 200, 700, 16, 4, True),  # prompt after an existing context
    (1, 130, 0, 16, 8, False),   # kv_mul 2, no gate
    (1, 97, 3, 32, 1, True),     # kv_mul 32: 4 rows per workgroup
    (1, 64, 0, 8, 8, False),     # kv_mul 1
    (3, 33, 31, 16, 4, True),    # short rows straddling a 32-key block
])
def test_prefill128_full_vs_oracle(gpu, orc, n_seq, n_tok, pos_0, nq, nkv, gate):
    rng = np.random.default_rng(n_tok * 11 + pos_0 + nq + nkv)
    q, k16, v16, g, got = run(gpu, rng, n_seq, n_tok, pos_0, nq, nkv, gate=gate)
    for s in range(n_seq):
        want = oracle(orc, q, k16, v16, g, s, pos_0, 0, 0, nq, nkv)
        parity(got[s], want, what=f"prefill128 s={s} n={n_tok} pos0={pos_0} {nq}q/{nkv}kv gate={gate}")


@pytest.mark.parametrize("n_tok,pos_0,window,kv_pos0", [
    (700, 0, 256, 0),        # window edge moves through the prompt
    (400, 1000, 256, 745),   # linear copy of the window before the prompt
    (300, 100, 256, 0),      # window longer than the context so far
    (250, 40, 33, 8),        # odd window, not a block multiple
    (100, 500, 1, 500),      # window 1: each row sees only its own key
    (64, 9, 300, 0),         # window never binds
])
def test_prefill128_window_vs_oracle(gpu, orc, n_tok, pos_0, window, kv_pos0):
    assert kv_pos0 <= t_start(pos_0, window)
    rng = np.random.default_rng(n_tok + pos_0 + window)
    q, k16, v16, g, got = run(gpu, rng, 2, n_tok, pos_0, 16, 4, window=window, kv_pos0=kv_pos0)
    for s in range(2):
        want = oracle(orc, q, k16, v16, g, s, pos_0, kv_pos0, window, 16, 4)
        parity(got[s], want, what=f"prefill128 window={window} s={s} n={n_tok} pos0={pos_0} kv_pos0={kv_pos0}")
    if window == 1:
        # softmax over one key: the output is V of the row's own position
        # times the gate, whatever the scores
        v = f16_to_f32(v16)[:, pos_0 - kv_pos0:]
        want = np.repeat(v, 4, axis=2) * sigmoid(g)[..., None]
        assert np.allclose(got, want, rtol=1e-6, atol=1e-7)


def test_prefill128_lfm3_full_size_sampled(gpu, orc):
    """The bench workload (B 4 x 4096, 16q/4kv d128, gated full layer):
    sampled rows against the oracle, every output a gate-scaled convex
    combination of V rows, and row 0 equal to V[0] times its gate."""
    rng = np.random.default_rng(4128)
    q, k16, v16, g, got = run(gpu, rng, 4, 4096, 0, 16, 4)
    rows = [0, 1, 31, 32, 127, 128, 1000, 2047, 4095]
    for s in range(4):
        want = oracle(orc, q, k16, v16, g, s, 0, 0, 0, 16, 4, rows=rows)
        parity(got[s][rows], want, what=f"prefill128 B4x4096 s={s} sampled")
    vmax = np.abs(f16_to_f32(v16)).max()
    assert np.all(np.isfinite(got)) and np.abs(got).max() <= vmax + 1e-3
    v0 = f16_to_f32(v16[:, 0])
    assert np.allclose(got[:, 0], np.repeat(v0, 4, axis=1) * sigmoid(g[:, 0])[..., None], atol=1e-6)


def test_prefill128_swa_full_size_sampled(gpu, orc):
    """An LFM3 sliding-window layer at the bench shape: window 4096 - 512
    over B 2 x 4096 rows, sampled rows against the oracle."""
    rng = np.random.default_rng(4129)
    window = 3584
    q, k16, v16, g, got = run(gpu, rng, 2, 4096, 0, 16, 4, window=window)
    rows = [0, 3583, 3584, 3600, 4095]
    for s in range(2):
        want = oracle(orc, q, k16, v16, g, s, 0, 0, window, 16, 4, rows=rows)
        parity(got[s][rows], want, what=f"prefill128 swa B2x4096 s={s} sampled")


@pytest.mark.parametrize("pattern", ["rising", "spike", "falling", "sunk", "outside"])
def test_prefill128_lazy_max(gpu, orc, pattern):
    """Score patterns that exercise the lazy running max: scores climbing by
    tens of log2 units ("rising"), isolated huge scores ("spike"), a large
    first block ("falling"), a first block whose scores all lie below -128
    log2 units, where exp2(-m) overflows ("sunk"), and huge scores on keys
    just outside each row's window ("outside": they must get no weight)."""
    la = gpu
    rng = np.random.default_rng({"rising": 1, "spike": 2, "falling": 3, "sunk": 4, "outside": 5}[pattern])
    n_tok, nq, nkv = 300, 16, 4
    window = 64 if pattern == "outside" else 0
    q = rng.standard_normal((1, n_tok, nq, HD), dtype=np.float32)
    k = rng.standard_normal((1, n_tok, nkv, HD), dtype=np.float32) * 0.5
    u = rng.standard_normal(HD).astype(np.float32)
    u /= np.linalg.norm(u)
    q += 3.0 * u
    t = np.arange(n_tok, dtype=np.float32)
    amp = {"rising": 0.25 * t,
           "spike": np.where(t % 97 == 40, 60.0, 0.0),
           "falling": np.where(t < 64, 40.0, 0.0),
           "sunk": np.where(t < 32, -400.0, 0.0),
           "outside": np.where(t % 50 == 7, 80.0, 0.0)}[pattern].astype(np.float32)
    k += amp[None, :, None, None] * u
    k16 = f16(k)
    v16 = f16(rng.standard_normal((1, n_tok, nkv, HD), dtype=np.float32))
    _, _, _, g, got = run(la, rng, 1, n_tok, 0, nq, nkv, window=window, q=q, k16=k16, v16=v16)
    want = oracle(orc, q, k16, v16, g, 0, 0, 0, window, nq, nkv)
    parity(got[0], want, what=f"prefill128 lazy max {pattern}")


@pytest.mark.parametrize("n_tok,pos_0,window,kv_pos0,gate", [(300, 0, 0, 0, True), (250, 40, 33, 8, True),
                                                             (200, 700, 0, 0, False)])
def test_prefill_ext_head_dim_64(gpu, orc, n_tok, pos_0, window, kv_pos0, gate):
    """The same entry point at head_dim 64 (32q/8kv): windows and the gate
    for head_dim-64 layers (the LFM2 prompt path, lfm_hip_prefill_f16, has
    neither and keeps its 64-column kernel)."""
    rng = np.random.default_rng(n_tok + window + 64)
    q, k16, v16, g, got = run(gpu, rng, 2, n_tok, pos_0, 32, 8, window=window, kv_pos0=kv_pos0, gate=gate, hd=64)
    for s in range(2):
        want = oracle(orc, q, k16, v16, g, s, pos_0, kv_pos0, window, 32, 8)
        parity(got[s], want, what=f"prefill ext d64 window={window} s={s} n={n_tok} pos0={pos_0}")


@pytest.mark.parametrize("chain", [2, 3, 5])
@pytest.mark.parametrize("n_tok,pos_0,window,kv_pos0,nq,nkv,hd", [
    (700, 0, 256, 0, 16, 4, 128),     # LFM3 SWA heads: 22 query tiles, ragged last chain
    (400, 1000, 256, 745, 16, 4, 128),  # prompt after a cached window (linear copy)
    (250, 40, 33, 8, 16, 8, 128),     # odd window, kv_mul 2 (64-position tiles)
    (300, 5, 100, 0, 32, 8, 64),      # head_dim 64
    (100, 500, 1, 500, 16, 4, 128),   # window 1
])
def test_prefill128_window_chains(gpu, orc, chain, n_tok, pos_0, window, kv_pos0, nq, nkv, hd):
    """Sliding-window prefill with `chain` consecutive query tiles per
    workgroup (their key blocks streamed through one LDS ring, the next
    tile's first blocks fetched while the current one finishes): outputs
    bit-identical to one tile per workgroup (same blocks, same order, same
    arithmetic per tile) and within tolerance of the oracle."""
    la = gpu
    rng = np.random.default_rng(n_tok + window + chain)
    with la.tuning(prefill_chain=1):
        q, k16, v16, g, one = run(la, rng, 2, n_tok, pos_0, nq, nkv, window=window, kv_pos0=kv_pos0, hd=hd)
    with la.tuning(prefill_chain=chain):
        _, _, _, _, got = run(la, rng, 2, n_tok, pos_0, nq, nkv, window=window, kv_pos0=kv_pos0, q=q, k16=k16,
                              v16=v16, hd=hd, gate_values=g)
    assert np.array_equal(got.view(np.uint32), one.view(np.uint32)), "chained tiles differ from single tiles"
    for s in range(2):
        want = oracle(orc, q, k16, v16, g, s, pos_0, kv_pos0, window, nq, nkv)
        parity(got[s], want, what=f"prefill window={window} chain={chain} s={s} n={n_tok} d{hd}")


def test_prefill128_swa256_bench_shape_sampled(gpu, orc):
    """The bench's sliding-window workload (B 4 x 4096, 16q/4kv d128, window
    256, gate) with the automatic chain length: rows at chain and tile
    boundaries against the oracle, and bit-identical to one tile per
    workgroup."""
    la = gpu
    rng = np.random.default_rng(4256)
    q, k16, v16, g, got = run(la, rng, 4, 4096, 0, 16, 4, window=256)
    with la.tuning(prefill_chain=1):
        _, _, _, _, one = run(la, rng, 4, 4096, 0, 16, 4, window=256, q=q, k16=k16, v16=v16, gate_values=g)
    assert np.array_equal(got.view(np.uint32), one.view(np.uint32))
    rows = [0, 31, 32, 127, 128, 255, 256, 257, 1023, 1024, 2047, 2048, 4064, 4095]
    for s in (0, 3):
        want = oracle(orc, q, k16, v16, g, s, 0, 0, 256, 16, 4, rows=rows)
        parity(got[s][rows], want, what=f"prefill128 swa256 B4x4096 s={s} sampled")
