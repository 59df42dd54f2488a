"""GPU parity of the production LFM2 prologue (LFM_PROLOGUE_TABLE): the
QK-RMSNorm + RoPE that lfm2_forward.c (decode) and lfm2_prefill_batch.c
(speculative verify, prompt prefill) run -- lfm2_qk_norm_and_rope /
lfm2_qk_norm_and_rope_table (tools/lfm2_forward.c:775-830,
tools/lfm2_prefill_batch.c:826-893) with lfm2_rmsnorm's sum order
(tools/lfm2_forward.c:669-684) and the float-angle table of the state
initialisers (tools/lfm2_prefill_batch.c:727-736).  Every check is against
the oracle's TABLE restatement, which tests/test_oracle.py pins bit for bit
to those reference functions compiled from source.  Positions 1023, 8191 and
32767 are where the float-angle and double-angle tables drift apart."""
import numpy as np
import pytest

from helpers import f16, parity, rand_kv

pytestmark = pytest.mark.gpu

EPS = 1e-5
POSITIONS = (1023, 8191, 32767)


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


@pytest.mark.parametrize("hd", [64, 128, 48, 40, 16])
def test_qk_norm_rope_table_bit_exact(gpu, orc, hd):
    """lfm_hip_qk_norm_rope with LFM_PROLOGUE_TABLE: Q (fp32 in place) and K
    (RNE fp16 store) bit for bit at every position, with and without norm
    weights, on inputs spanning six orders of magnitude; head dims with
    scalar tails in the norm (40) and the rotation (48, 40, 16)."""
    la = gpu
    rng = np.random.default_rng(70 + hd)
    n_heads = 12
    cos, sin = la.rope_table_lfm2(32768, hd, 1e6)
    ocos, osin = orc.rope_table_lfm2(32768, hd, 1e6)
    assert np.array_equal(cos.view(np.uint32), ocos.view(np.uint32))
    cd, sd = dev(la, cos), dev(la, sin)
    for pos in (0,) + POSITIONS:
        for norm in (True, False):
            x = (rng.standard_normal(n_heads * hd) * rng.choice([1e-3, 1.0, 40.0], n_heads * hd)).astype(np.float32)
            w = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32) if norm else None
            wd = None if w is None else dev(la, w)
            xq = dev(la, x)
            la.qk_norm_rope(xq, None, n_heads, hd, wd, EPS, cd, sd, pos, prologue=la.PROLOGUE_TABLE)
            want = orc.qk_norm_rope(x, n_heads, hd, w, EPS, ocos[pos], osin[pos], table=True)
            assert np.array_equal(xq.numpy().view(np.uint32), want.view(np.uint32)), (hd, pos, norm)
            k16 = la.DeviceArray.zeros(n_heads * hd, np.uint16)
            la.qk_norm_rope(dev(la, x), k16, n_heads, hd, wd, EPS, cd, sd, pos, prologue=la.PROLOGUE_TABLE)
            want_k = orc.qk_norm_rope(x, n_heads, hd, w, EPS, ocos[pos], osin[pos], store_f16=True, table=True)
            assert np.array_equal(k16.numpy(), want_k), (hd, pos, norm)


def _table_case(la, orc, seed, n_rows, pos0, fused, nq=32, nkv=8, hd=64):
    """Config-2 heads; one sequence per position in pos0, n_rows rows each:
    the fused step (fused=True) or the batched prologue then varlen attention.
    Returns (outputs, K caches, rotated q of the two-launch path or None)."""
    rng = np.random.default_rng(seed)
    pos0 = np.asarray(pos0, np.uint32)
    n_seq = len(pos0)
    rows = int(pos0.max()) + n_rows
    cos, sin = la.rope_table_lfm2(rows, hd, 1e6)
    k0 = [rand_kv(rng, int(p) + n_rows, nkv, hd) for p in pos0]
    v0 = [rand_kv(rng, int(p) + n_rows, nkv, hd) for p in pos0]
    q = rng.standard_normal((n_seq, n_rows, nq, hd), dtype=np.float32) * 2
    k = rng.standard_normal((n_seq, n_rows, nkv, hd), dtype=np.float32) * 2
    v = rng.standard_normal((n_seq, n_rows, nkv, hd), dtype=np.float32)
    qw = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
    kd, vd = [dev(la, x) for x in k0], [dev(la, x) for x in v0]
    kt, vt, pd = la.pointer_table(kd), la.pointer_table(vd), dev(la, pos0)
    qd = dev(la, q)
    out = la.DeviceArray.zeros(q.shape, np.float32)
    args = (dev(la, qw), dev(la, kw), EPS, dev(la, cos), dev(la, sin))
    if fused:
        la.gqa_f16_step(qd, dev(la, k), dev(la, v), None, True, kt, vt, pd, out, n_seq, n_rows, rows, nq, nkv, hd,
                        *args, prologue=la.PROLOGUE_TABLE)
        qr = None
    else:
        la.qkv_prologue(qd, dev(la, k), dev(la, v), kt, vt, pd, n_seq, n_rows, nq, nkv, hd, *args,
                        prologue=la.PROLOGUE_TABLE)
        la.gqa_f16_varlen(qd, None, True, kt, vt, pd, out, n_seq, n_rows, rows, nq, nkv, hd)
        qr = qd.numpy()
    inputs = dict(q=q, k=k, v=v, qw=qw, kw=kw, k0=k0, v0=v0, cos=cos, sin=sin)
    return out.numpy(), [x.numpy() for x in kd], [x.numpy() for x in vd], qr, inputs


@pytest.mark.parametrize("n_rows", [1, 8])
def test_step_table_prologue_bit_exact_rows(gpu, orc, n_rows):
    """The fused step (one attention launch) with LFM_PROLOGUE_TABLE at
    positions 1023, 8191 and 32767 (decode, and the B = 8 verify of
    tools/lfm2_speculative_pld.c:388-461): every new K row bit-identical to
    the oracle's, V rows RNE, every other cache row untouched; the rotated Q
    of the two-launch path bit-identical to the oracle's and, on one plan,
    the fused step's outputs bit-identical to that path's (so the fused
    kernel's Q is the oracle's too); outputs of the automatic plan within
    2e-3 / 1e-3 of the oracle's attention."""
    la = gpu
    pos0 = [p - (n_rows - 1) for p in POSITIONS]
    # one plan for both paths (the fused and plain kernels differ in
    # occupancy, so the automatic balanced plan may cut their keys apart)
    with la.tuning("grid"):
        got1, _, _, _, _ = _table_case(la, orc, 91 + n_rows, n_rows, pos0, True)
        got2, kc2, _, qr, _ = _table_case(la, orc, 91 + n_rows, n_rows, pos0, False)
    assert np.array_equal(got1.view(np.uint32), got2.view(np.uint32)), "fused step vs prologue + attention"
    got, kc, vc, _, inp = _table_case(la, orc, 91 + n_rows, n_rows, pos0, True)  # automatic plan
    nq, nkv, hd = 32, 8, 64
    ocos, osin = orc.rope_table_lfm2(32768, hd, 1e6)
    for s, p0 in enumerate(pos0):
        kh, vh = inp["k0"][s].copy(), inp["v0"][s].copy()
        qs = np.empty((n_rows, nq, hd), np.float32)
        for r in range(n_rows):
            p = p0 + r
            qs[r] = orc.qk_norm_rope(inp["q"][s, r], nq, hd, inp["qw"], EPS, ocos[p], osin[p],
                                     table=True).reshape(nq, hd)
            kh[p] = orc.qk_norm_rope(inp["k"][s, r], nkv, hd, inp["kw"], EPS, ocos[p], osin[p], store_f16=True,
                                     table=True).reshape(nkv, hd)
            vh[p] = f16(inp["v"][s, r])
        assert np.array_equal(qr[s].view(np.uint32), qs.view(np.uint32)), f"Q rows at {p0}"
        assert np.array_equal(kc[s], kh), f"K rows at {p0}"
        assert np.array_equal(kc2[s], kh), f"K rows at {p0} (two launches)"
        assert np.array_equal(vc[s], vh), f"V rows at {p0}"
        want = orc.lfm3_online_gqa_f16(qs, None, kh, vh, n_rows, p0, 0, p0 + n_rows, nq, nkv, hd)
        parity(got[s], want, what=f"table step pos0 {p0} rows {n_rows}")


def test_table_and_fast_prologues_differ(gpu, orc):
    """The two prologue forms store different K bits at position 32767 on the
    same raw inputs (the tables differ by ~1e-3 there), so a step that
    ignored the form would fail the bit-exact checks above."""
    la = gpu
    rng = np.random.default_rng(5)
    hd, n_heads, pos = 64, 8, 32767
    x = rng.standard_normal(n_heads * hd).astype(np.float32)
    w = dev(la, (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32))
    outs = []
    for form, (c, s) in ((la.PROLOGUE_FAST, la.rope_lut_lfm2(32768, hd, 1e6)),
                         (la.PROLOGUE_TABLE, la.rope_table_lfm2(32768, hd, 1e6))):
        k16 = la.DeviceArray.zeros(n_heads * hd, np.uint16)
        la.qk_norm_rope(dev(la, x), k16, n_heads, hd, w, EPS, dev(la, c), dev(la, s), pos, prologue=form)
        outs.append(k16.numpy())
    assert np.count_nonzero(outs[0] != outs[1]) > 0


def test_context_table_prologue(gpu, orc):
    """lfm_attn_ctx with prologue = LFM_PROLOGUE_TABLE (an LFM2-1.2B attention
    layer, 32q/8kv d64, max_seq 32768): history imported, then decode steps at
    positions 1023, 8191 and 32767 and an 8-row verify chunk ending at 8191;
    the K rows the context writes are bit-identical to the oracle's TABLE
    prologue and the outputs within 2e-3 / 1e-3 of the oracle's attention.
    Then a 600-row prompt prefill (prologue launch + MFMA prefill) whose
    cache rows are bit-identical to the oracle's."""
    la = gpu
    rng = np.random.default_rng(33)
    nq, nkv, hd, max_seq = 32, 8, 64, 32768
    ctx = la.EngineContext(1, nq, nkv, hd, max_seq, EPS, rope_base=1e6, prologue=la.PROLOGUE_TABLE)
    qn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
    ctx.set_norms(0, qn, kn)
    ocos, osin = orc.rope_table_lfm2(max_seq, hd, 1e6)
    K = rand_kv(rng, max_seq, nkv, hd).reshape(max_seq, nkv * hd)
    V = rand_kv(rng, max_seq, nkv, hd).reshape(max_seq, nkv * hd)
    ctx.kv_import(0, 0, K, V)
    for pos_0, B in ((1023, 1), (8184, 8), (32767, 1)):
        q = rng.standard_normal((B, nq, hd), dtype=np.float32) * 2
        k = rng.standard_normal((B, nkv, hd), dtype=np.float32) * 2
        v = rng.standard_normal((B, nkv, hd), dtype=np.float32)
        got = ctx.forward(0, pos_0, q, k, v)
        qr = np.empty_like(q)
        for b in range(B):
            p = pos_0 + b
            qr[b] = orc.qk_norm_rope(q[b], nq, hd, qn, EPS, ocos[p], osin[p], table=True).reshape(nq, hd)
            K[p] = orc.qk_norm_rope(k[b], nkv, hd, kn, EPS, ocos[p], osin[p], store_f16=True, table=True)
            V[p] = f16(v[b]).reshape(-1)
        kh, vh = ctx.kv_export(0, pos_0, B)
        assert np.array_equal(kh.reshape(B, -1), K[pos_0:pos_0 + B]), f"K rows at {pos_0}"
        assert np.array_equal(vh.reshape(B, -1), V[pos_0:pos_0 + B])
        want = orc.lfm3_online_gqa_f16(qr, None, K, V, B, pos_0, 0, max_seq, nq, nkv, hd)
        parity(got, want, what=f"context table prologue pos {pos_0} B {B}")
    # prompt prefill of 600 rows at positions 4000 .. 4599
    n, p0 = 600, 4000
    q = rng.standard_normal((n, nq, hd), dtype=np.float32) * 2
    k = rng.standard_normal((n, nkv, hd), dtype=np.float32) * 2
    v = rng.standard_normal((n, nkv, hd), dtype=np.float32)
    got = ctx.prefill(0, p0, q, k, v).reshape(n, nq, hd)
    for r in range(n):
        K[p0 + r] = orc.qk_norm_rope(k[r], nkv, hd, kn, EPS, ocos[p0 + r], osin[p0 + r], store_f16=True, table=True)
        V[p0 + r] = f16(v[r]).reshape(-1)
    kh, vh = ctx.kv_export(0, p0, n)
    assert np.array_equal(kh.reshape(n, -1), K[p0:p0 + n]) and np.array_equal(vh.reshape(n, -1), V[p0:p0 + n])
    for r in (0, 257, 599):
        p = p0 + r
        qr = orc.qk_norm_rope(q[r], nq, hd, qn, EPS, ocos[p], osin[p], table=True).reshape(1, nq, hd)
        want = orc.lfm3_online_gqa_f16(qr, None, K, V, 1, p, 0, max_seq, nq, nkv, hd)
        # the MFMA prefill enters q * scale * log2(e) as fp16
        parity(got[r], want, what=f"context table prefill row {r}")
    ctx.close()
