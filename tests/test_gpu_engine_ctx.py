"""GPU parity of the engine context (device-resident KV, prologue + attention
per layer step) against an oracle emulation of the reference forward stacks:
lfm2_forward_gqa_fast / lfm2_forward_gqa_batch (LFM2) and
lfm3_forward_token_internal / lfm3_forward_batch_core (LFM3)."""
import numpy as np
import pytest

from helpers import f16, parity

pytestmark = pytest.mark.gpu


class RefEngine:
    """Host KV caches + oracle kernels, called the way the reference engine
    calls its CPU kernels (K/V of all B rows written, then attention)."""

    def __init__(self, orc, nq, nkv, hd, max_seq, eps, luts, norms, swa=None, cap=0):
        self.orc, self.nq, self.nkv, self.hd, self.eps = orc, nq, nkv, hd, eps
        self.luts, self.norms, self.swa = luts, norms, swa
        self.caps = [cap if (swa and swa[l]) else max_seq for l in range(len(luts))]
        self.K = [np.zeros((c, nkv * hd), np.uint16) for c in self.caps]
        self.V = [np.zeros((c, nkv * hd), np.uint16) for c in self.caps]

    def step(self, layer, pos_0, q, k, v, gate_logits, window):
        o, nq, nkv, hd = self.orc, self.nq, self.nkv, self.hd
        cos, sin = self.luts[layer]
        qn, kn = self.norms[layer]
        B = q.shape[0]
        qr = np.empty_like(q)
        for b in range(B):
            p = pos_0 + b
            slot = p % self.caps[layer] if window else p
            qr[b] = o.qk_norm_rope(q[b], nq, hd, qn, self.eps, cos[p], sin[p]).reshape(nq, hd)
            self.K[layer][slot] = o.qk_norm_rope(k[b], nkv, hd, kn, self.eps, cos[p], sin[p], store_f16=True)
            self.V[layer][slot] = f16(v[b]).reshape(-1)
        g = None
        if gate_logits is not None:
            g = (1.0 / (1.0 + np.exp(-gate_logits.astype(np.float64)))).astype(np.float32)
        return o.lfm3_online_gqa_f16(qr, g, self.K[layer], self.V[layer], B, pos_0, window,
                                     self.caps[layer], nq, nkv, hd)


def schedule(n_steps, rng, max_b=8):
    pos, out = 0, []
    for i in range(n_steps):
        b = int(rng.choice([1, 1, 1, 3, max_b]))
        out.append((pos, b))
        pos += b
    return out


def test_lfm2_session(gpu, orc):
    la = gpu
    rng = np.random.default_rng(2024)
    nq, nkv, hd, max_seq, eps = 32, 8, 64, 512, 1e-5
    ctx = la.EngineContext(2, nq, nkv, hd, max_seq, eps, rope_base=1e6)
    norms = []
    for l in range(2):
        qn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        kn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        ctx.set_norms(l, qn, kn)
        norms.append((qn, kn))
    lut = orc.rope_lut_lfm2(max_seq, hd, 1e6)
    ref = RefEngine(orc, nq, nkv, hd, max_seq, eps, [lut, lut], norms)
    for pos_0, B in schedule(40, rng):
        for layer in range(2):
            q = rng.standard_normal((B, nq, hd), dtype=np.float32) * 2
            k = rng.standard_normal((B, nkv, hd), dtype=np.float32) * 2
            v = rng.standard_normal((B, nkv, hd), dtype=np.float32) * 0.5
            got = ctx.forward(layer, pos_0, q, k, v)
            want = ref.step(layer, pos_0, q, k, v, None, 0)
            parity(got, want, what=f"lfm2 layer {layer} pos {pos_0} B {B}")
    last = pos_0 + B
    for layer in range(2):
        kh, vh = ctx.kv_export(layer, 0, last)
        assert np.array_equal(vh, ref.V[layer][:last])
        d = np.abs(kh.astype(np.int32) - ref.K[layer][:last].astype(np.int32))
        assert d.max() <= 1 and np.count_nonzero(d) <= d.size // 500
    ctx.close()


def test_lfm3_session_swa_ring_partial_rope_gate(gpu, orc):
    """Two LFM3 layers: a sliding-window layer (window 16 in a 24-slot ring,
    RoPE base 1e4) and a full layer with partial RoPE (rope_freqs 1 / 1e30) and
    base 1e6; sigmoid output gate; positions run through several ring wraps."""
    la = gpu
    rng = np.random.default_rng(3)
    nq, nkv, hd, max_seq, eps, win, cap = 16, 4, 128, 256, 1e-5, 16, 24
    rf = np.array([1.0] * 32 + [1e30] * 32, np.float32)
    ctx = la.EngineContext(2, nq, nkv, hd, max_seq, eps, rope_base=1e6, lfm3=True,
                           sliding_window=win, swa_cap=cap, layer_is_swa=[1, 0],
                           rope_base_swa=1e4, rope_dim=hd, rope_freqs=rf)
    norms = []
    for l in range(2):
        qn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        kn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        ctx.set_norms(l, qn, kn)
        norms.append((qn, kn))
    luts = [orc.rope_lut_lfm3(max_seq, hd, hd, 1e4, None), orc.rope_lut_lfm3(max_seq, hd, hd, 1e6, rf)]
    ref = RefEngine(orc, nq, nkv, hd, max_seq, eps, luts, norms, swa=[1, 0], cap=cap)
    for pos_0, B in schedule(30, rng):
        for layer in range(2):
            q = rng.standard_normal((B, nq, hd), dtype=np.float32) * 2
            k = rng.standard_normal((B, nkv, hd), dtype=np.float32) * 2
            v = rng.standard_normal((B, nkv, hd), dtype=np.float32) * 0.5
            g = rng.standard_normal((B, nq)).astype(np.float32)
            got = ctx.forward(layer, pos_0, q, k, v, g)
            want = ref.step(layer, pos_0, q, k, v, g, win if layer == 0 else 0)
            parity(got, want, what=f"lfm3 layer {layer} pos {pos_0} B {B}")
    assert pos_0 + B > 3 * cap  # the ring wrapped several times
    ctx.close()


def test_kv_export_import_round_trip(gpu):
    """Checkpoint / .lfmcache data path: export, import into a fresh context,
    continue decoding -- bit-identical outputs and caches."""
    la = gpu
    rng = np.random.default_rng(11)
    nq, nkv, hd, max_seq = 32, 8, 64, 300
    a = la.EngineContext(1, nq, nkv, hd, max_seq)
    b = la.EngineContext(1, nq, nkv, hd, max_seq)
    for pos in range(50):
        a.forward(0, pos, rng.standard_normal((1, nq, hd), dtype=np.float32),
                  rng.standard_normal((1, nkv, hd), dtype=np.float32),
                  rng.standard_normal((1, nkv, hd), dtype=np.float32))
    kh, vh = a.kv_export(0, 0, 50)
    b.kv_import(0, 0, kh, vh)
    kh2, vh2 = b.kv_export(0, 0, 50)
    assert np.array_equal(kh, kh2) and np.array_equal(vh, vh2)
    q = rng.standard_normal((1, nq, hd), dtype=np.float32)
    k = rng.standard_normal((1, nkv, hd), dtype=np.float32)
    v = rng.standard_normal((1, nkv, hd), dtype=np.float32)
    assert np.array_equal(a.forward(0, 50, q, k, v), b.forward(0, 50, q, k, v))
    a.close()
    b.close()


def test_context_range_errors(gpu):
    la = gpu
    with pytest.raises(la.LfmAttnError) as e:    # 16 + 8 - 1 > 20 ring slots: refused at creation
        la.EngineContext(1, 16, 4, 128, 64, lfm3=True, sliding_window=16, swa_cap=20, layer_is_swa=[1])
    assert e.value.status == -1
    ctx = la.EngineContext(1, 16, 4, 128, 64, lfm3=True, sliding_window=16, swa_cap=23,
                           layer_is_swa=[1])
    z = np.zeros((8, 16, 128), np.float32)
    zk = np.zeros((8, 4, 128), np.float32)
    with pytest.raises(la.LfmAttnError) as e:
        ctx.forward(0, 60, z[:8], zk[:8], zk[:8])  # past max_seq
    assert e.value.status == -2
    out = ctx.forward(0, 0, z[:8], zk[:8], zk[:8])  # 8 rows on a window + 7 ring
    assert np.all(out == 0.0)
    ctx.close()


def test_context_prefill_matches_chunked_steps(gpu, orc):
    """lfm_attn_ctx_prefill of a 600-token prompt after 37 cached tokens (LFM2
    layer, 32q/8kv d64: the MFMA prefill path) against the same prompt run
    through the step 8 rows at a time, as lfm2_forward_batch does: caches
    bit-identical (same prologue), outputs within the attention tolerance;
    sampled rows also against the oracle engine."""
    la = gpu
    rng = np.random.default_rng(21)
    nq, nkv, hd, max_seq, eps = 32, 8, 64, 1024, 1e-5
    a = la.EngineContext(1, nq, nkv, hd, max_seq, eps, rope_base=1e6)
    b = la.EngineContext(1, nq, nkv, hd, max_seq, eps, rope_base=1e6)
    qn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
    for c in (a, b):
        c.set_norms(0, qn, kn)
    pre = 37
    q0 = rng.standard_normal((pre, nq, hd), dtype=np.float32)
    k0 = rng.standard_normal((pre, nkv, hd), dtype=np.float32)
    v0 = rng.standard_normal((pre, nkv, hd), dtype=np.float32)
    for c in (a, b):
        for p in range(0, pre, 8):
            c.forward(0, p, q0[p:p + 8], k0[p:p + 8], v0[p:p + 8])
    n = 600
    q = rng.standard_normal((n, nq, hd), dtype=np.float32) * 2
    k = rng.standard_normal((n, nkv, hd), dtype=np.float32) * 2
    v = rng.standard_normal((n, nkv, hd), dtype=np.float32) * 0.5
    got = a.prefill(0, pre, q, k, v).reshape(n, nq, hd)
    want = np.concatenate([b.forward(0, pre + p, q[p:p + 8], k[p:p + 8], v[p:p + 8]).reshape(-1, nq, hd)
                           for p in range(0, n, 8)])
    parity(got, want, what="ctx prefill vs chunked steps")
    ka, va = a.kv_export(0, 0, pre + n)
    kb, vb = b.kv_export(0, 0, pre + n)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    # sampled rows against the oracle on the exported caches
    lut = orc.rope_lut_lfm2(max_seq, hd, 1e6)
    for r in (0, 1, 299, n - 1):
        p = pre + r
        qr = orc.qk_norm_rope(q[r], nq, hd, qn, eps, lut[0][p], lut[1][p])
        ref_o = orc.online_gqa_f16(qr, ka[:p + 1], va[:p + 1], nq, nq // nkv, nkv * hd, p, 1.0 / 8.0)
        parity(got[r].reshape(-1), ref_o, what=f"ctx prefill row {r} vs oracle")
    a.close()
    b.close()


@pytest.mark.parametrize("win,cap,pre,n", [(16, 24, 0, 45), (16, 24, 21, 45), (256, 264, 300, 700)])
def test_context_prefill_lfm3_layers(gpu, orc, win, cap, pre, n):
    """LFM3 prompt prefill through the head_dim-128 MFMA kernel: a
    sliding-window layer (the window before the prompt copied out of the
    ring into a linear buffer, the ring refilled afterwards) and a gated full
    layer with partial RoPE, after `pre` cached tokens.  Against the same
    prompt run through the step 8 rows at a time (lfm3_forward_batch_core's
    batches): every cache slot bit-identical (same prologue, same ring state),
    outputs within the attention tolerance; and against the oracle engine."""
    la = gpu
    rng = np.random.default_rng(22 + pre + win)
    nq, nkv, hd, max_seq, eps = 16, 4, 128, 1024, 1e-5
    rf = np.array([1.0] * 32 + [1e30] * 32, np.float32)
    mk = lambda: la.EngineContext(2, nq, nkv, hd, max_seq, eps, rope_base=1e6, lfm3=True, sliding_window=win,
                                  swa_cap=cap, layer_is_swa=[1, 0], rope_base_swa=1e4, rope_dim=hd,
                                  rope_freqs=rf)
    a, b = mk(), mk()
    norms = []
    for layer in range(2):
        qn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        kn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        norms.append((qn, kn))
        for c in (a, b):
            c.set_norms(layer, qn, kn)
    luts = [orc.rope_lut_lfm3(max_seq, hd, hd, 1e4, None), orc.rope_lut_lfm3(max_seq, hd, hd, 1e6, rf)]
    ref = RefEngine(orc, nq, nkv, hd, max_seq, eps, luts, norms, swa=[1, 0], cap=cap)
    mk_rows = lambda m: (rng.standard_normal((m, nq, hd), dtype=np.float32) * 2,
                         rng.standard_normal((m, nkv, hd), dtype=np.float32) * 2,
                         rng.standard_normal((m, nkv, hd), dtype=np.float32) * 0.5,
                         rng.standard_normal((m, nq)).astype(np.float32))
    for layer in range(2):
        window = win if layer == 0 else 0
        q, k, v, g = mk_rows(pre)
        for p in range(0, pre, 8):
            sl = slice(p, p + 8)
            for c in (a, b):
                c.forward(layer, p, q[sl], k[sl], v[sl], g[sl])
            ref.step(layer, p, q[sl], k[sl], v[sl], g[sl], window)
        q, k, v, g = mk_rows(n)
        got = a.prefill(layer, pre, q, k, v, g).reshape(n, nq, hd)
        want = np.concatenate([b.forward(layer, pre + p, q[p:p + 8], k[p:p + 8], v[p:p + 8], g[p:p + 8])
                               .reshape(-1, nq, hd) for p in range(0, n, 8)])
        parity(got, want, what=f"ctx prefill layer {layer} vs chunked steps")
        oracle = np.concatenate([ref.step(layer, pre + p, q[p:p + 8], k[p:p + 8], v[p:p + 8], g[p:p + 8], window)
                                 .reshape(-1, nq, hd) for p in range(0, n, 8)])
        parity(got, oracle, what=f"ctx prefill layer {layer} vs oracle engine")
        slots = cap if layer == 0 else pre + n
        ka, va = a.kv_export(layer, 0, slots)
        kb, vb = b.kv_export(layer, 0, slots)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"layer {layer}: caches differ"
    a.close()
    b.close()


def test_context_prefill_chunked_layers(gpu):
    """Shapes the MFMA prefill kernels do not take (a gated head_dim-64
    layer) and prompts of at most 8 rows run the step in chunks of 8:
    bit-identical to calling the step that way."""
    la = gpu
    rng = np.random.default_rng(23)
    for nq, nkv, hd, n, gated in ((16, 4, 64, 45, True), (16, 4, 128, 8, True)):
        a = la.EngineContext(1, nq, nkv, hd, 256, 1e-5, rope_base=1e6)
        b = la.EngineContext(1, nq, nkv, hd, 256, 1e-5, rope_base=1e6)
        q = rng.standard_normal((n, nq, hd), dtype=np.float32)
        k = rng.standard_normal((n, nkv, hd), dtype=np.float32)
        v = rng.standard_normal((n, nkv, hd), dtype=np.float32)
        g = rng.standard_normal((n, nq)).astype(np.float32) if gated else None
        got = a.prefill(0, 0, q, k, v, g)
        want = np.concatenate([b.forward(0, p, q[p:p + 8], k[p:p + 8], v[p:p + 8],
                                         None if g is None else g[p:p + 8]) for p in range(0, n, 8)])
        assert np.array_equal(got, want)
        with pytest.raises(la.LfmAttnError) as e:
            a.prefill(0, 250, np.zeros((8, nq, hd), np.float32), np.zeros((8, nkv, hd), np.float32),
                      np.zeros((8, nkv, hd), np.float32))
        assert e.value.status == -2
        a.close()
        b.close()
