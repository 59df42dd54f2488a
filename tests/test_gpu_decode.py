"""GPU parity of the decode / verify / LFM3 attention kernels against the CPU
oracle (the restatement of the reference workers), through the C-ABI."""

import numpy as np
import pytest

from helpers import f16, f16_to_f32, parity, plan_overrides, rand_kv, softmax_attention_f64

pytestmark = pytest.mark.gpu


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


# ---- A1: tools/lfm2_kernels_fast.c:700-810 --------------------------------------------------

def test_a1_reference_inputs(gpu, orc):
    """Inputs of tests/test_kernels_fast.c:175-236 (16q/4kv, d64, seq 128, pos 37)."""
    la = gpu
    nq, nkv, hd, seq, pos = 16, 4, 64, 128, 37
    kv = nkv * hd
    q = np.cos(np.arange(nq * hd, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    i = np.arange(seq * kv, dtype=np.float32)
    k16 = f16(np.sin(i * np.float32(0.01)))
    v16 = f16(np.cos(i * np.float32(0.02)))
    out = la.DeviceArray.zeros(nq * hd, np.float32)
    la.online_gqa_f16(dev(la, q), dev(la, k16), dev(la, v16), out, nq, nq // nkv, kv, pos, 0.125)
    want = orc.online_gqa_f16(q, k16, v16, nq, nq // nkv, kv, pos)
    parity(out.numpy(), want, what="A1 reference inputs")
    # the reference's own gate for this case: FP16 online vs FP32 two-pass within 5e-4
    two_pass = orc.gqa_heads(q, nq, nq // nkv, hd, kv, pos, k32=np.sin(i * np.float32(0.01)),
                             v32=np.cos(i * np.float32(0.02)))
    assert np.abs(out.numpy() - two_pass).max() < 5e-4


@pytest.mark.parametrize("pos", [0, 1, 15, 31, 32, 33, 63, 64, 100, 511, 1023])
def test_a1_cfg1_positions(gpu, orc, pos):
    """BASELINE config 1 shape (16q/8kv, d64, ctx up to 1024) at sub-tile edges."""
    la = gpu
    rng = np.random.default_rng(100 + pos)
    nq, nkv, hd = 16, 8, 64
    q = rng.standard_normal(nq * hd, dtype=np.float32)
    k16 = rand_kv(rng, 1024, nkv, hd)
    v16 = rand_kv(rng, 1024, nkv, hd)
    out = la.DeviceArray.zeros(nq * hd, np.float32)
    la.online_gqa_f16(dev(la, q), dev(la, k16), dev(la, v16), out, nq, 2, nkv * hd, pos, 0.125)
    want = orc.online_gqa_f16(q, k16, v16, nq, 2, nkv * hd, pos)
    parity(out.numpy(), want, what=f"A1 cfg1 pos={pos}")


def test_a1_float64_closed_form(gpu):
    """Independent of the oracle: textbook softmax in float64."""
    la = gpu
    rng = np.random.default_rng(7)
    nq, nkv, hd, pos = 32, 8, 64, 777
    q = rng.standard_normal(nq * hd, dtype=np.float32)
    k16 = rand_kv(rng, pos + 1, nkv, hd)
    v16 = rand_kv(rng, pos + 1, nkv, hd)
    out = la.DeviceArray.zeros(nq * hd, np.float32)
    la.online_gqa_f16(dev(la, q), dev(la, k16), dev(la, v16), out, nq, 4, nkv * hd, pos, 0.125)
    kf, vf = f16_to_f32(k16), f16_to_f32(v16)
    want = np.concatenate([softmax_attention_f64(q[h * hd:(h + 1) * hd], kf[:, h // 4], vf[:, h // 4],
                                                 0.125) for h in range(nq)])
    parity(out.numpy(), want, max_abs=1e-5, rel_l2=1e-5, what="A1 vs float64")


# ---- A2: tools/lfm2_threadpool.c:764-931 ----------------------------------------------------

@pytest.mark.parametrize("hd", [64, 128, 16, 32])
def test_a2_f16_branch(gpu, orc, hd):
    la = gpu
    rng = np.random.default_rng(hd)
    nq, nkv, pos, seq = 8, 2, 90, 100
    kv = nkv * hd
    q = rng.standard_normal(nq * hd, dtype=np.float32)
    k16 = rand_kv(rng, seq, nkv, hd)
    v16 = rand_kv(rng, seq, nkv, hd)
    init = np.full(nq * hd, 7.0, np.float32)  # dims the reference leaves untouched keep this
    out = dev(la, init)
    la.gqa_heads(dev(la, q), None, None, dev(la, k16), dev(la, v16), out, nq, nq // nkv, hd, kv,
                 seq, pos)
    want = orc.gqa_heads(q, nq, nq // nkv, hd, kv, pos, k16=k16, v16=v16, out=init)
    got = out.numpy()
    parity(got, want, what=f"A2 f16 hd={hd}")
    if hd > 64:  # tools/lfm2_threadpool.c:783 writes only 64 dims
        assert np.all(got.reshape(nq, hd)[:, 64:] == 7.0)


def test_a2_f32_two_pass(gpu, orc):
    la = gpu
    rng = np.random.default_rng(3)
    nq, nkv, hd, seq, pos = 16, 4, 64, 64, 50
    kv = nkv * hd
    q = rng.standard_normal(nq * hd, dtype=np.float32)
    k = rng.standard_normal(seq * kv, dtype=np.float32) * np.float32(0.5)
    v = rng.standard_normal(seq * kv, dtype=np.float32) * np.float32(0.5)
    out = la.DeviceArray.zeros(nq * hd, np.float32)
    la.gqa_heads(dev(la, q), dev(la, k), dev(la, v), None, None, out, nq, 4, hd, kv, seq, pos)
    want = orc.gqa_heads(q, nq, 4, hd, kv, pos, k32=k, v32=v)
    parity(out.numpy(), want, max_abs=1e-5, rel_l2=1e-5, what="A2 fp32 two-pass")


# ---- A3: tools/lfm3_engine.c:851-1204 -------------------------------------------------------

def test_a3_reference_ring_wrap(gpu, orc):
    """tests/test_lfm3.c:170-251: 8q/2kv d128, window 16, cap 24, 42 positions
    through the ring wrap, gates 0.25+0.08h, checked against the exact
    two-pass SWA softmax times the gate (reference gate 1e-4)."""
    la = gpu
    nq, nkv, hd, win, cap = 8, 2, 128, 16, 24
    kv = nkv * hd
    k_ring = np.zeros((cap, kv), np.uint16)
    v_ring = np.zeros((cap, kv), np.uint16)
    k_lin = np.zeros((64, kv), np.float32)
    v_lin = np.zeros((64, kv), np.float32)
    gate = (np.float32(0.25) + np.float32(0.08) * np.arange(nq, dtype=np.float32)).astype(np.float32)
    kd, vd = la.DeviceArray((cap, kv), np.uint16), la.DeviceArray((cap, kv), np.uint16)
    gd = dev(la, gate)
    out = la.DeviceArray.zeros(nq * hd, np.float32)
    worst = 0.0
    for pos in range(42):
        slot = pos % cap
        i = np.arange(kv, dtype=np.float32)
        k_ring[slot] = f16(np.float32(0.4) * np.sin((np.float32(pos * 19) + i) * np.float32(0.11)))
        v_ring[slot] = f16(np.float32(0.5) * np.cos((np.float32(pos * 23) + i) * np.float32(0.09)))
        k_lin[pos], v_lin[pos] = f16_to_f32(k_ring[slot]), f16_to_f32(v_ring[slot])
        q = (np.float32(0.3) * np.sin((np.float32(pos * 13) + np.arange(nq * hd, dtype=np.float32))
                                      * np.float32(0.07))).astype(np.float32)
        kd.upload(k_ring)
        vd.upload(v_ring)
        la.lfm3_online_gqa_f16_dispatch(dev(la, q), gd, kd, vd, out, 1, pos, win, cap, nq, nkv, hd)
        got = out.numpy()
        want = orc.lfm3_online_gqa_f16(q, gate, k_ring, v_ring, 1, pos, win, cap, nq, nkv, hd)
        parity(got, want, what=f"A3 wrap pos={pos}")
        t0 = max(0, pos + 1 - win)
        for h in range(nq):
            kvh = h // (nq // nkv)
            exact = softmax_attention_f64(q[h * hd:(h + 1) * hd], k_lin[t0:pos + 1, kvh * hd:(kvh + 1) * hd],
                                          v_lin[t0:pos + 1, kvh * hd:(kvh + 1) * hd],
                                          1.0 / np.sqrt(np.float32(hd))) * gate[h]
            worst = max(worst, float(np.abs(got[h * hd:(h + 1) * hd] - exact).max()))
    assert worst < 1e-4, worst


@pytest.mark.parametrize("B,pos_0,win,cap", [(3, 30, 16, 24), (8, 1000, 256, 264), (8, 5, 256, 264),
                                              (4, 2000, 0, 4096), (8, 250, 256, 264)])
def test_a3_batched_rows(gpu, orc, B, pos_0, win, cap):
    """B rows per call (prefill / verify of lfm3_forward_batch_core, :1918-2055)."""
    la = gpu
    rng = np.random.default_rng(B * 1000 + pos_0)
    nq, nkv, hd = 16, 4, 128
    k16 = rand_kv(rng, cap, nkv, hd)
    v16 = rand_kv(rng, cap, nkv, hd)
    q = rng.standard_normal((B, nq, hd), dtype=np.float32)
    gate = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, nq)).astype(np.float32)))
    gate = gate.astype(np.float32)
    out = la.DeviceArray.zeros(q.shape, np.float32)
    la.lfm3_online_gqa_f16_dispatch(dev(la, q), dev(la, gate), dev(la, k16), dev(la, v16), out, B,
                                    pos_0, win, cap, nq, nkv, hd)
    want = orc.lfm3_online_gqa_f16(q, gate, k16, v16, B, pos_0, win, cap, nq, nkv, hd)
    parity(out.numpy(), want, what=f"A3 B={B} pos0={pos_0} win={win} cap={cap}")


# ---- multi-sequence batches (3, 5) ---------------------------------------

def _varlen_case(la, orc, rng, n_seq, n_rows, nq, nkv, hd, ctx, win=0, cap=0, gate=False,
                 slots=None):
    """ctx[s] = keys before the batch rows; rows are positions ctx[s] .. ctx[s]+n_rows-1."""
    pos0 = np.asarray(ctx, np.uint32)
    caches_k, caches_v, kd, vd = [], [], [], []
    for s in range(n_seq):
        n_slots = slots if slots else int(pos0[s]) + n_rows
        k = rand_kv(rng, n_slots, nkv, hd)
        v = rand_kv(rng, n_slots, nkv, hd)
        caches_k.append(k)
        caches_v.append(v)
        kd.append(dev(la, k))
        vd.append(dev(la, v))
    q = rng.standard_normal((n_seq, n_rows, nq, hd), dtype=np.float32)
    g = rng.standard_normal((n_seq, n_rows, nq)).astype(np.float32) if gate else None
    out = la.DeviceArray.zeros(q.shape, np.float32)
    max_keys = int(win + n_rows - 1) if win else int(pos0.max() + n_rows)
    la.gqa_f16_varlen(dev(la, q), None if g is None else dev(la, g), True, la.pointer_table(kd),
                      la.pointer_table(vd), dev(la, pos0), out, n_seq, n_rows, max_keys, nq, nkv,
                      hd, win, cap)
    got = out.numpy()
    want = np.empty_like(got)
    for s in range(n_seq):
        gs = None if g is None else (1.0 / (1.0 + np.exp(-g[s]))).astype(np.float32)
        want[s] = orc.lfm3_online_gqa_f16(q[s], gs, caches_k[s], caches_v[s], n_rows, int(pos0[s]),
                                          win, cap if cap else int(pos0[s]) + n_rows, nq, nkv,
                                          hd).reshape(n_rows, nq, hd)
    return got, want


def test_varlen_cfg2_reduced(gpu, orc):
    """Config 2 shape (32q/8kv d64), 8 sequences with ctx uniform in [512, 2048]."""
    rng = np.random.default_rng(22)
    ctx = rng.integers(512, 2049, size=8) - 1
    got, want = _varlen_case(gpu, orc, rng, 8, 1, 32, 8, 64, ctx)
    parity(got, want, what="varlen cfg2 reduced")


def test_varlen_verify_cfg3_reduced(gpu, orc):
    """Config 3 shape: 8 causal rows over ctx 4096 + drafts, 32q/8kv d64, 4 sequences."""
    rng = np.random.default_rng(33)
    got, want = _varlen_case(gpu, orc, rng, 4, 8, 32, 8, 64, [4096] * 4)
    parity(got, want, what="verify cfg3 reduced")


@pytest.mark.parametrize("cap", [256, 264])
def test_varlen_lfm3_swa_cfg5(gpu, orc, cap):
    """Config 5 SWA layer: B32, 16q/4kv d128, window 256 in a ring of `cap`
    slots, write head at position 1000, sigmoid gate from logits."""
    rng = np.random.default_rng(cap)
    got, want = _varlen_case(gpu, orc, rng, 32, 1, 16, 4, 128, [1000] * 32, win=256, cap=cap,
                             gate=True, slots=cap)
    parity(got, want, what=f"lfm3 swa cap={cap}")


def test_split_count_invariance(gpu, orc):
    """Size-independent property: the key chunk per workgroup (and so the
    number of splits merged) must not change results beyond fp32 rounding."""
    la = gpu
    outs = []
    for chunk in (1000000, 96, 32, 160, 64):
        with la.tuning(chunk=chunk):
            got, want = _varlen_case(la, orc, np.random.default_rng(5), 3, 2, 32, 8, 64,
                                     [3000, 100, 2047])
        parity(got, want, what=f"chunk={chunk}")
        outs.append(got)
    for o in outs[1:]:
        assert np.abs(outs[0] - o).max() < 1e-5


def test_repeated_calls_shared_workspace(gpu, orc):
    """Back-to-back calls of different batch shapes reuse (and grow) the split
    workspace; every call stays correct."""
    rng = np.random.default_rng(6)
    for i, (n_seq, n_rows, ctx) in enumerate([(4, 1, 5000), (2, 8, 700), (4, 1, 5000),
                                              (7, 1, 300), (1, 3, 9000)]):
        got, want = _varlen_case(gpu, orc, rng, n_seq, n_rows, 32, 8, 64, [ctx] * n_seq)
        parity(got, want, what=f"repeat {i}")


def plan_tol(n_rows, nq, nkv):
    """Agreement expected between two plans of the same batch: fp32 rounding
    with one 16-column tile (P enters P.V split hi + lo, ~exact); with more
    query columns P enters as one fp16 value, and plans that cut the keys at
    other points (so with other running maxima) round it differently."""
    return 1e-5 if n_rows * (nq // nkv) <= 16 else 2e-4


@pytest.mark.parametrize("hd,nq,nkv,n_rows,n_seq", [(64, 32, 8, 1, 130), (128, 16, 4, 1, 9),
                                                    (64, 32, 8, 8, 5), (64, 16, 8, 1, 1)])
def test_balanced_plan_matches_grid_plan(gpu, orc, hd, nq, nkv, n_rows, n_seq):
    """The balanced split (every workgroup takes the same number of key
    tiles, cut at sequence and head-group boundaries) and the fixed-chunk grid
    (plan override "grid") both match the oracle on ragged batches; also with
    96-key shares (many more segments than sequences)."""
    la = gpu
    rng = np.random.default_rng(n_seq * 31 + hd)
    ctx = [int(c) for c in rng.integers(0, 3000, size=n_seq)]
    if n_seq > 1:
        ctx[0], ctx[-1] = 0, 2999  # one-key and longest sequences
    outs = []
    for env in ({"LFM_ATTN_PLAN": "balanced"}, {"LFM_ATTN_PLAN": "grid"},
                {"LFM_ATTN_PLAN": "balanced", "LFM_ATTN_CHUNK": "96"}):
        with plan_overrides(la, env):
            got, want = _varlen_case(la, orc, np.random.default_rng(4), n_seq, n_rows, nq, nkv, hd,
                                     ctx)
        parity(got, want, what=f"{env}")
        outs.append(got)
    for o in outs[1:]:
        assert np.abs(outs[0] - o).max() < plan_tol(n_rows, nq, nkv)


@pytest.mark.parametrize("hd,nq,nkv,n_rows,n_seq,max_ctx,win,cap,gate,default", [
    (64, 16, 8, 1, 1, 300, 0, 0, False, "wg"),       # config-1 heads, short context: the default small-batch form
    (64, 32, 8, 8, 2, 400, 0, 0, False, "balanced-dma"),  # verify rows (32 query columns; two sequences: balanced, LDS-streamed)
    (64, 32, 4, 8, 1, 1000, 0, 0, False, "wg"),      # 64 query columns (four-wave workgroups, 2 splits)
    (128, 16, 4, 1, 3, 500, 0, 0, False, "balanced"),  # LFM3 head_dim 128 (ragged: balanced by default)
    (128, 16, 4, 1, 1, 900, 200, 208, True, "wg"),   # SWA ring (window 200, 208 slots) + gate: 4 splits
    (64, 32, 8, 1, 2, 3000, 0, 0, False, "balanced"),  # forced: more planned splits than waves, chunks lengthened
])
def test_workgroup_merge_plan(gpu, orc, hd, nq, nkv, n_rows, n_seq, max_ctx, win, cap, gate, default):
    """Small batches take one workgroup per (sequence, KV head) whose waves
    split the keys and merge in place (k_splitkv_wg, the "wg" override
    forces it); it matches the oracle and the two-kernel grid, and with no override
    the automatic rule picks the expected form (lfm_attn_last_plan)."""
    la = gpu
    rng = np.random.default_rng(max_ctx + n_seq + hd)
    ctx = [int(c) for c in rng.integers(1, max_ctx, size=n_seq)]
    ctx[0] = max_ctx - 1
    outs = []
    for env in ({}, {"LFM_ATTN_PLAN": "wg"}, {"LFM_ATTN_PLAN": "grid"}):
        with plan_overrides(la, env):
            got, want = _varlen_case(la, orc, np.random.default_rng(9), n_seq, n_rows, nq, nkv, hd, ctx, win=win,
                                     cap=cap, gate=gate, slots=cap or None)
            plan = la.last_plan()
        parity(got, want, what=f"{env}")
        assert plan == (default if not env else env["LFM_ATTN_PLAN"]), f"{env}: plan {plan}"
        outs.append(got)
    assert np.abs(outs[1] - outs[2]).max() < plan_tol(n_rows, nq, nkv)
