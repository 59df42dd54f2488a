"""The allocation-free decode entry point (lfm_hip_gqa_f16_varlen_noalloc):
same kernels and plan as lfm_hip_gqa_f16_varlen, split partials in the
library's fixed device array.  Checked against that entry point (bit for
bit) and the oracle, on two calls in a row, the second smaller; and a batch
whose partials exceed the array is rejected before anything runs."""
import numpy as np
import pytest

from helpers import parity, rand_kv

pytestmark = pytest.mark.gpu


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def _case(la, orc, rng, n_seq, n_rows, nq, nkv, hd, ctx, win=0, cap=0, gate=False):
    pos0 = np.asarray(ctx, np.uint32)
    ks, vs = [], []
    for s in range(n_seq):
        n_slots = cap if cap else int(pos0[s]) + n_rows
        ks.append(rand_kv(rng, n_slots, nkv, hd))
        vs.append(rand_kv(rng, n_slots, nkv, hd))
    kd, vd = [dev(la, k) for k in ks], [dev(la, v) for v in vs]
    q = rng.standard_normal((n_seq, n_rows, nq, hd), dtype=np.float32)
    g = rng.standard_normal((n_seq, n_rows, nq)).astype(np.float32) if gate else None
    args = (dev(la, q), None if g is None else dev(la, g), True, la.pointer_table(kd), la.pointer_table(vd),
            dev(la, pos0))
    keys = int(win + n_rows - 1) if win else int(pos0.max() + n_rows)
    outs = []
    for fn in (la.gqa_f16_varlen_noalloc, la.gqa_f16_varlen):
        out = la.DeviceArray.zeros(q.shape, np.float32)
        fn(*args, out, n_seq, n_rows, keys, nq, nkv, hd, win, cap)
        outs.append(out.numpy())
    assert np.array_equal(outs[0], outs[1]), "no-alloc entry differs from lfm_hip_gqa_f16_varlen"
    for s in range(n_seq):
        gs = None if g is None else (1.0 / (1.0 + np.exp(-g[s]))).astype(np.float32)
        want = orc.lfm3_online_gqa_f16(q[s], gs, ks[s], vs[s], n_rows, int(pos0[s]), win,
                                       cap if cap else int(pos0[s]) + n_rows, nq, nkv, hd)
        parity(outs[0][s], want, what=f"noalloc seq {s}")


def test_noalloc_matches_varlen_two_calls(gpu, orc):
    la = gpu
    rng = np.random.default_rng(77)
    # first call: ragged B48 decode (balanced plan, many partial slots)
    ctx = rng.integers(1, 6000, size=48)
    ctx[0] = 0
    _case(la, orc, rng, 48, 1, 32, 8, 64, ctx)
    # second call, smaller: 3 sequences x 8 verify rows (the array keeps the
    # first call's contents)
    _case(la, orc, rng, 3, 8, 32, 8, 64, [700, 1500, 33])
    # LFM3 sliding-window ring with a gate (grid plan)
    _case(la, orc, rng, 4, 1, 16, 4, 128, [1000] * 4, win=256, cap=264, gate=True)


def test_noalloc_rejects_oversized_batch(gpu):
    """1024 sequences x 8 rows need far more than 32 MiB of partials: the call
    returns LFM_ATTN_E_SCRATCH and leaves the output untouched."""
    la = gpu
    n_seq, n_rows, nq, nkv, hd = 1024, 8, 32, 8, 64
    k = la.DeviceArray.zeros((64 + n_rows, nkv, hd), np.uint16)
    v = la.DeviceArray.zeros((64 + n_rows, nkv, hd), np.uint16)
    kt, vt = la.pointer_table([k] * n_seq), la.pointer_table([v] * n_seq)
    pos0 = dev(la, np.full(n_seq, 64, np.uint32))
    q = la.DeviceArray.zeros((n_seq, n_rows, nq, hd), np.float32)
    init = np.full((n_seq, n_rows, nq, hd), 3.0, np.float32)
    out = dev(la, init)
    with pytest.raises(la.LfmAttnError) as e:
        la.gqa_f16_varlen_noalloc(q, None, True, kt, vt, pos0, out, n_seq, n_rows, 64 + n_rows, nq, nkv, hd)
    assert e.value.status == -7
    assert np.array_equal(out.numpy(), init)
