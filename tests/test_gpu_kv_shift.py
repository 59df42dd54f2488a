"""GPU parity of attention-sink eviction (lfm_hip_kv_cache_shift_sinks,
lfm_hip_lfm3_kv_cache_shift_sinks, lfm_attn_ctx_shift_sinks) against the
oracle restatement of tools/lfm2_runtime_features.c:744-833 / 1055-1163:
every cache byte bit-exact, same new position."""
import numpy as np
import pytest

from helpers import parity
from test_gpu_engine_ctx import RefEngine
from test_kv_shift_oracle import RF_PARTIAL, copies, lut2, lut3, rand_cache

pytestmark = pytest.mark.gpu


def upload(la, caches):
    return [None if c is None else la.DeviceArray.from_numpy(c) for c in caches]


def download(arrs):
    return [None if a is None else a.numpy() for a in arrs]


def assert_caches_equal(got, want):
    for g, w in zip(got, want):
        assert (g is None and w is None) or np.array_equal(g, w)


@pytest.mark.parametrize("pos,n_sink,n_discard", [
    (2040, 64, 1024),  # engine trigger (pos + 8 >= max_seq, n_discard = max_seq / 2): one move
    (1000, 16, 100),   # overlapping move: 9 chunks of <= 100 rows
    (513, 0, 1),       # one-row shift: 512 single-row chunks
    (300, 64, 500),    # no-op (pos <= n_sink + n_discard)
])
def test_lfm2_shift_vs_oracle(gpu, orc, pos, n_sink, n_discard):
    la = gpu
    rng = np.random.default_rng(pos + n_discard)
    rows, hd = 2048, 64
    nkv = [8, 0, 8, 4]
    K = [rand_cache(rng, rows, n * hd) if n else None for n in nkv]
    V = [rand_cache(rng, rows, n * hd, 1.0) if n else None for n in nkv]
    lut = lut2(orc, rows)
    dK, dV = upload(la, K), upload(la, V)
    dc, ds = la.DeviceArray.from_numpy(lut[0]), la.DeviceArray.from_numpy(lut[1])
    new = la.kv_cache_shift_sinks(dK, dV, nkv, hd, dc, ds, rows, pos, n_sink, n_discard)
    la.sync()
    want = orc.kv_shift_sinks_lfm2(K, V, nkv, hd, lut, pos, n_sink, n_discard)
    assert new == want
    assert_caches_equal(download(dK), K)
    assert_caches_equal(download(dV), V)


@pytest.mark.parametrize("cap,win,pos,n_sink,n_discard", [
    (264, 256, 32760, 64, 16384),  # LFM3 engine trigger at max_seq 32768, engine ring
    (256, 256, 1000, 64, 500),     # BASELINE cfg 5 ring
    (24, 16, 60, 4, 10),           # window reaches the sinks
    (40, 16, 39, 2, 30),           # new position below the window
])
def test_lfm3_shift_vs_oracle(gpu, orc, cap, win, pos, n_sink, n_discard):
    la = gpu
    rng = np.random.default_rng(cap * 7 + pos)
    hd, nkv = 128, 4
    rows_full = pos + 8
    kinds = [1, 2, 0, 2]
    K = [rand_cache(rng, rows_full, nkv * hd), rand_cache(rng, cap, nkv * hd), None,
         rand_cache(rng, cap, nkv * hd)]
    V = [rand_cache(rng, rows_full, nkv * hd), rand_cache(rng, cap, nkv * hd), None,
         rand_cache(rng, cap, nkv * hd)]
    lf = lut3(orc, rows_full, hd, 1e6, RF_PARTIAL)
    lw = lut3(orc, rows_full, hd, 1e4)
    dK, dV = upload(la, K), upload(la, V)
    dl = [la.DeviceArray.from_numpy(x) for x in (*lf, *lw)]
    n_kv = [nkv, nkv, 0, nkv]
    new = la.lfm3_kv_cache_shift_sinks(dK, dV, n_kv, kinds, hd, dl[0], dl[1], rows_full, dl[2],
                                       dl[3], rows_full, win, cap, pos, n_sink, n_discard)
    la.sync()
    want = orc.kv_shift_sinks_lfm3(K, V, n_kv, kinds, hd, lf, lw, win, cap, pos, n_sink, n_discard)
    assert new == want == pos - n_discard
    assert_caches_equal(download(dK), K)
    assert_caches_equal(download(dV), V)


def test_lfm2_context_decode_shift_decode(gpu, orc):
    """Engine session: decode to within 8 of max_seq, evict with sinks
    (src/lfm2_api.c:871-891 trigger and arguments), keep decoding; outputs and
    caches follow the oracle engine doing the same."""
    la = gpu
    rng = np.random.default_rng(77)
    nq, nkv, hd, max_seq, eps, n_sink = 16, 8, 64, 96, 1e-5, 8
    ctx = la.EngineContext(2, nq, nkv, hd, max_seq, eps, rope_base=1e6)
    norms = []
    for l in range(2):
        qn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        kn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        ctx.set_norms(l, qn, kn)
        norms.append((qn, kn))
    lut = lut2(orc, max_seq)
    ref = RefEngine(orc, nq, nkv, hd, max_seq, eps, [lut, lut], norms)

    def step(pos, B):
        for layer in range(2):
            q = rng.standard_normal((B, nq, hd), dtype=np.float32) * 2
            k = rng.standard_normal((B, nkv, hd), dtype=np.float32) * 2
            v = rng.standard_normal((B, nkv, hd), dtype=np.float32) * 0.5
            got = ctx.forward(layer, pos, q, k, v)
            want = ref.step(layer, pos, q, k, v, None, 0)
            parity(got, want, what=f"layer {layer} pos {pos} B {B}")

    pos = 0
    while pos + 8 < max_seq:
        B = int(rng.choice([1, 3, 8]))
        B = min(B, max_seq - 8 - pos)
        step(pos, B)
        pos += B
    # the device caches before eviction (keys may differ from the oracle
    # engine's in the last fp16 bit: fp32 norm summation order)
    pre = [ctx.kv_export(layer, 0, pos) for layer in range(2)]
    dev_k = [np.ascontiguousarray(np.vstack([k, np.zeros((max_seq - pos, k.shape[1]), np.uint16)]))
             for k, _ in pre]
    dev_v = [np.ascontiguousarray(np.vstack([v, np.zeros((max_seq - pos, v.shape[1]), np.uint16)]))
             for _, v in pre]
    new = ctx.shift_sinks(pos, n_sink, max_seq // 2)
    want_pos = orc.kv_shift_sinks_lfm2(dev_k, dev_v, [nkv, nkv], hd, lut, pos, n_sink, max_seq // 2)
    assert orc.kv_shift_sinks_lfm2(ref.K, ref.V, [nkv, nkv], hd, lut, pos, n_sink,
                                   max_seq // 2) == want_pos
    assert new == want_pos == pos - max_seq // 2
    for layer in range(2):
        kh, vh = ctx.kv_export(layer, 0, new)
        assert np.array_equal(kh, dev_k[layer][:new]) and np.array_equal(vh, dev_v[layer][:new])
        assert np.array_equal(vh, ref.V[layer][:new])
        # continue from identical caches
        ctx.kv_import(layer, 0, ref.K[layer][:new], ref.V[layer][:new])
    for _ in range(6):
        step(new, 1)
        new += 1
    ctx.close()


def test_lfm3_context_shift_matches_oracle(gpu, orc):
    """LFM3 context (one full layer with partial RoPE, one SWA layer in a
    24-slot ring): caches imported, evicted on the device, compared bit-exact
    with the oracle eviction of the same caches."""
    la = gpu
    rng = np.random.default_rng(5)
    nq, nkv, hd, max_seq, win, cap = 16, 4, 128, 128, 16, 24
    ctx = la.EngineContext(2, nq, nkv, hd, max_seq, 1e-5, rope_base=1e6, lfm3=True,
                           sliding_window=win, swa_cap=cap, layer_is_swa=[0, 1],
                           rope_base_swa=1e4, rope_dim=hd, rope_freqs=RF_PARTIAL)
    K = [rand_cache(rng, max_seq, nkv * hd), rand_cache(rng, cap, nkv * hd)]
    V = [rand_cache(rng, max_seq, nkv * hd), rand_cache(rng, cap, nkv * hd)]
    for layer in range(2):
        ctx.kv_import(layer, 0, K[layer], V[layer])
    pos, n_sink = 120, 8
    new = ctx.shift_sinks(pos, n_sink, max_seq // 2)
    lf = lut3(orc, max_seq, hd, 1e6, RF_PARTIAL)
    lw = lut3(orc, max_seq, hd, 1e4)
    want = orc.kv_shift_sinks_lfm3(K, V, [nkv, nkv], [1, 2], hd, lf, lw, win, cap, pos, n_sink,
                                   max_seq // 2)
    assert new == want == pos - max_seq // 2
    for layer, rows in ((0, max_seq), (1, cap)):
        kh, vh = ctx.kv_export(layer, 0, rows)
        assert np.array_equal(kh, K[layer]) and np.array_equal(vh, V[layer])
    ctx.close()
