"""GPU parity of the attention step with the prologue fused into the
attention kernel (lfm_hip_gqa_f16_step): raw q/k/v rows in; QK-RMSNorm +
RoPE of q and of the new keys, the RNE fp16 K/V store at each row's slot, and
the attention out -- against the oracle's prologue (A4/A5) followed by its
attention (A1/A3), as the reference runs them
(tools/lfm2_kernels_fast.c:1046-1066, tools/lfm2_prefill_batch.c:1029-1092,
tools/lfm3_engine.c:1885-1896, 2006-2022)."""

import numpy as np
import pytest

from helpers import f16, parity, plan_overrides, rand_kv

pytestmark = pytest.mark.gpu

EPS = 1e-5


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def _luts(la, orc, hd, lut_kind, rows):
    if lut_kind == "lfm2":
        return la.rope_lut_lfm2(rows, hd, 1e6), orc.rope_lut_lfm2(rows, hd, 1e6)
    if lut_kind == "swa":
        return la.rope_lut_lfm3(rows, hd, hd, 1e4, None), orc.rope_lut_lfm3(rows, hd, hd, 1e4, None)
    rf = np.array([1.0] * (hd // 4) + [1e30] * (hd // 4), np.float32)
    return la.rope_lut_lfm3(rows, hd, hd, 1e6, rf), orc.rope_lut_lfm3(rows, hd, hd, 1e6, rf)


def _step_case(la, orc, seed, n_seq, n_rows, nq, nkv, hd, pos0, win=0, cap=0, gate=False, norm=True,
               lut_kind="lfm2", env=None):
    rng = np.random.default_rng(seed)
    pos0 = np.asarray(pos0, np.uint32)
    slots = [cap if win else int(p) + n_rows for p in pos0]
    k0 = [rand_kv(rng, n, nkv, hd) for n in slots]
    v0 = [rand_kv(rng, n, nkv, hd) for n in slots]
    kd, vd = [dev(la, k) for k in k0], [dev(la, v) for v in v0]
    q = rng.standard_normal((n_seq, n_rows, nq, hd), dtype=np.float32)
    k = rng.standard_normal((n_seq, n_rows, nkv, hd), dtype=np.float32)
    v = rng.standard_normal((n_seq, n_rows, nkv, hd), dtype=np.float32)
    qw = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    kw = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    g = rng.standard_normal((n_seq, n_rows, nq)).astype(np.float32) if gate else None
    rows = int(pos0.max()) + n_rows
    (cos, sin), (ocos, osin) = _luts(la, orc, hd, lut_kind, rows)
    qd = dev(la, q)
    out = la.DeviceArray.zeros(q.shape, np.float32)
    keys = win + n_rows - 1 if win else rows
    env = env or {}
    with plan_overrides(la, env):
        la.gqa_f16_step(qd, dev(la, k), dev(la, v), None if g is None else dev(la, g), True, la.pointer_table(kd),
                        la.pointer_table(vd), dev(la, pos0), out, n_seq, n_rows, keys, nq, nkv, hd,
                        None if qw is None else dev(la, qw), None if kw is None else dev(la, kw), EPS,
                        dev(la, cos), dev(la, sin), win, cap)
    got = out.numpy()
    assert np.array_equal(qd.numpy(), q), "the step must leave q unchanged"
    for s in range(n_seq):
        kh, vh = k0[s].copy(), v0[s].copy()
        qs = np.empty((n_rows, nq, hd), np.float32)
        new_slots = []
        for r in range(n_rows):
            p = int(pos0[s]) + r
            slot = p % cap if win else p
            new_slots.append(slot)
            qs[r] = orc.qk_norm_rope(q[s, r], nq, hd, qw, EPS, ocos[p], osin[p]).reshape(nq, hd)
            kh[slot] = orc.qk_norm_rope(k[s, r], nkv, hd, kw, EPS, ocos[p], osin[p], store_f16=True).reshape(nkv, hd)
            vh[slot] = f16(v[s, r])
        gk, gv = kd[s].numpy(), vd[s].numpy()
        ulp = np.abs(gk.astype(np.int32) - kh.astype(np.int32))
        # bit-exact where the oracle follows the reference's AVX2 order (d64,
        # d128); other head dims sum in another order (1 ulp)
        assert ulp.max() <= (0 if hd in (64, 128) else 1), f"seq {s}: K rows differ by {ulp.max()} ulp"
        keep = np.ones(len(gk), bool)
        keep[new_slots] = False
        assert np.array_equal(gk[keep], k0[s][keep]), f"seq {s}: rows outside the new slots changed"
        assert np.array_equal(gv, vh), f"seq {s}: V rows"
        gs = None if g is None else (1.0 / (1.0 + np.exp(-g[s]))).astype(np.float32)
        want = orc.lfm3_online_gqa_f16(qs, gs, kh, vh, n_rows, int(pos0[s]), win, cap if win else slots[s], nq,
                                       nkv, hd)
        parity(got[s], want, what=f"step seq {s} pos0 {int(pos0[s])} {env}")
    return got


PLANS = [{}, {"LFM_ATTN_PLAN": "grid"}, {"LFM_ATTN_PLAN": "balanced", "LFM_ATTN_CHUNK": "96"},
         {"LFM_ATTN_PLAN": "wg"}, {"LFM_ATTN_PLAN": "grid", "LFM_ATTN_CHUNK": "32"}]


@pytest.mark.parametrize("env", PLANS)
def test_step_decode_ragged_lfm2(gpu, orc, env):
    """Config-2 heads (32q/8kv d64), 9 ragged sequences incl. a first token
    (position 0: the only key is the new one) under every plan."""
    pos0 = [0, 2999, 1, 31, 32, 33, 512, 1500, 2047]
    _step_case(gpu, orc, 11, 9, 1, 32, 8, 64, pos0, env=env)


@pytest.mark.parametrize("env", PLANS)
def test_step_verify_rows_straddling_splits(gpu, orc, env):
    """8 causal rows per sequence whose new keys cross a 32-key sub-tile and
    a split boundary (positions 956..963 around 960)."""
    _step_case(gpu, orc, 12, 3, 8, 32, 8, 64, [956, 4096, 20], env=env)


@pytest.mark.parametrize("env", [{}, {"LFM_ATTN_PLAN": "grid", "LFM_ATTN_CHUNK": "64"}])
def test_step_lfm3_swa_ring_gate(gpu, orc, env):
    """LFM3 SWA layer: 16q/4kv d128, window 256 in a 264-slot ring (window +
    8), 8 rows per sequence through the wrap, full RoPE theta 1e4, gate from
    logits (tools/lfm3_engine.c:1673, 1720-1723, 2006-2022)."""
    _step_case(gpu, orc, 13, 4, 8, 16, 4, 128, [1000, 250, 5, 263], win=256, cap=264, gate=True, lut_kind="swa",
               env=env)


@pytest.mark.parametrize("env", PLANS)
@pytest.mark.parametrize("n_rows,nq,nkv,pos0", [(8, 16, 4, [600]), (8, 16, 4, [380, 1000, 5]), (1, 32, 1, [600, 77]),
                                                 (3, 32, 4, [999])])
def test_step_lfm3_full_32_columns(gpu, orc, env, n_rows, nq, nkv, pos0):
    """head_dim 128 with 17..32 query columns per KV head (two 16-column
    tiles): an LFM3 full layer's 8-row chunk, 32 heads on one KV head, under
    every plan.  These instantiations of the workgroup-merge and balanced
    kernels returned wrong outputs while the segment bounds were held in
    VGPRs; the key loop now runs on wave-uniform bounds."""
    _step_case(gpu, orc, 18, len(pos0), n_rows, nq, nkv, 128, pos0, gate=True, lut_kind="partial", env=env)


def test_step_lfm3_full_partial_rope(gpu, orc):
    """LFM3 full layer: partial RoPE (pairs i < 32 rotate), gate, B = 1."""
    _step_case(gpu, orc, 14, 3, 1, 16, 4, 128, [2000, 0, 77], gate=True, lut_kind="partial")


def test_step_without_norm_weights(gpu, orc):
    """Layers without QK-norm weights: RoPE only."""
    _step_case(gpu, orc, 15, 2, 2, 16, 8, 64, [300, 40], norm=False)


def test_step_generic_head_dim(gpu, orc):
    """head_dim 32 (no split-KV kernel): prologue on a copy of q, then the
    generic kernel; same results."""
    _step_case(gpu, orc, 16, 2, 2, 8, 2, 32, [100, 7])


def test_step_matches_two_launch_path(gpu, orc):
    """The fused step and prologue-then-attention give bit-identical outputs
    and caches: both add the sum of squares in the reference's order and run
    the same attention plan."""
    la = gpu
    rng = np.random.default_rng(17)
    n_seq, nq, nkv, hd = 6, 32, 8, 64
    pos0 = np.array([0, 100, 4000, 63, 64, 2500], np.uint32)
    q = rng.standard_normal((n_seq, 1, nq, hd), dtype=np.float32)
    k = rng.standard_normal((n_seq, 1, nkv, hd), dtype=np.float32)
    v = rng.standard_normal((n_seq, 1, nkv, hd), dtype=np.float32)
    qw = dev(la, (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32))
    kw = dev(la, (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32))
    cos, sin = la.rope_lut_lfm2(4096, hd, 1e6)
    cd, sd = dev(la, cos), dev(la, sin)
    base_k = [rand_kv(rng, int(p) + 1, nkv, hd) for p in pos0]
    base_v = [rand_kv(rng, int(p) + 1, nkv, hd) for p in pos0]
    outs, caches = [], []
    for fused in (True, False):
        kd, vd = [dev(la, x) for x in base_k], [dev(la, x) for x in base_v]
        kt, vt, pd = la.pointer_table(kd), la.pointer_table(vd), dev(la, pos0)
        out = la.DeviceArray.zeros(q.shape, np.float32)
        qd = dev(la, q)
        if fused:
            la.gqa_f16_step(qd, dev(la, k), dev(la, v), None, True, kt, vt, pd, out, n_seq, 1, 4001, nq, nkv, hd,
                            qw, kw, EPS, cd, sd)
        else:
            la.qkv_prologue(qd, dev(la, k), dev(la, v), kt, vt, pd, n_seq, 1, nq, nkv, hd, qw, kw, EPS, cd, sd)
            la.gqa_f16_varlen(qd, None, True, kt, vt, pd, out, n_seq, 1, 4001, nq, nkv, hd)
        outs.append(out.numpy())
        caches.append([x.numpy() for x in kd])
    # same Q and K bits, same plan and kernels: identical outputs and caches
    assert np.array_equal(outs[0], outs[1])
    for a, b in zip(*caches):
        assert np.array_equal(a, b)
