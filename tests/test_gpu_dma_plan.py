"""GPU parity of the LDS-streamed balanced plan ("balanced-dma": k_splitkv_bal
with run_segment_dma -- head_dim 64 with up to 32 query columns, head_dim 128
with up to 16 -- K and V moved into each wave's LDS ring three 32-key
sub-tiles ahead) against the oracle's
lfm3_online_gqa_f16 (tools/lfm3_engine.c:851-946 semantics: rows at positions
ctx .. ctx + n_rows - 1 attend [t_start, pos]) and against the register
plan ("balanced") on the same batches."""
import numpy as np
import pytest

from helpers import parity
from test_gpu_decode import _varlen_case, plan_tol

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nq,nkv,n_rows,n_seq,max_ctx", [
    (32, 8, 1, 37, 3000),   # config-2 heads, ragged
    (32, 8, 8, 6, 4200),    # config-3 verify rows (two 16-column tiles)
    (16, 8, 1, 5, 1100),    # config-1 heads
    (16, 4, 8, 3, 900),     # 8 rows x 4 heads = 32 columns
    (16, 2, 2, 4, 700),     # two KV heads: waves 2, 3 of each workgroup idle
    (32, 8, 3, 9, 200),     # short sequences: fewer sub-tiles than the prefetch depth
    (8, 8, 1, 4, 5000),     # MHA, one column per KV head
])
def test_dma_plan_vs_oracle_and_register_plan(gpu, orc, nq, nkv, n_rows, n_seq, max_ctx):
    la = gpu
    rng = np.random.default_rng(max_ctx * 7 + n_seq * 3 + nq + nkv + n_rows)
    ctx = [int(c) for c in rng.integers(0, max_ctx, size=n_seq)]
    ctx[0] = 0                   # one key (or n_rows keys)
    ctx[-1] = max_ctx - 1
    if n_seq > 2:
        ctx[1] = 40              # one or two sub-tiles
    outs = {}
    for plan in ("balanced-dma", "balanced"):
        with la.tuning(plan):
            got, want = _varlen_case(la, orc, np.random.default_rng(5), n_seq, n_rows, nq, nkv, 64, ctx)
            assert la.last_plan() == plan
        parity(got, want, what=f"{plan} {nq}q/{nkv}kv rows={n_rows}")
        outs[plan] = got
    assert np.abs(outs["balanced-dma"] - outs["balanced"]).max() < plan_tol(n_rows, nq, nkv)


@pytest.mark.parametrize("chunk", [32, 96, 160])
def test_dma_plan_many_segments(gpu, orc, chunk):
    """Short shares (chunk override): each workgroup walks several segments
    of several sequences through the same LDS ring."""
    la = gpu
    rng = np.random.default_rng(chunk)
    ctx = [int(c) for c in rng.integers(0, 1500, size=11)]
    with la.tuning("balanced-dma", chunk=chunk):
        got, want = _varlen_case(la, orc, np.random.default_rng(8), 11, 2, 32, 8, 64, ctx)
        assert la.last_plan() == "balanced-dma"
    parity(got, want, what=f"balanced-dma chunk={chunk}")


@pytest.mark.parametrize("win,cap,n_rows", [(200, 208, 1), (256, 256, 1), (100, 107, 8)])
def test_dma_plan_window_ring(gpu, orc, win, cap, n_rows):
    """Sliding-window ring caches (slot = position % cap) with the output
    gate: sub-tiles that wrap the ring take the per-lane path."""
    la = gpu
    rng = np.random.default_rng(win + cap + n_rows)
    ctx = [int(c) for c in rng.integers(1, 2000, size=6)]
    ctx[0] = 5
    with la.tuning("balanced-dma"):
        got, want = _varlen_case(la, orc, np.random.default_rng(3), 6, n_rows, 32, 8, 64, ctx, win=win, cap=cap,
                                 gate=True, slots=cap)
        assert la.last_plan() == "balanced-dma"
    parity(got, want, what=f"balanced-dma window={win} cap={cap} rows={n_rows}")


@pytest.mark.parametrize("nq,nkv,n_rows,n_seq,max_ctx,win,cap,gate", [
    (16, 4, 1, 9, 5000, 0, 0, True),     # LFM3 full-layer heads, ragged, gate
    (16, 4, 4, 3, 1200, 0, 0, False),    # 4 rows x 4 heads = 16 columns
    (16, 4, 1, 7, 2000, 256, 264, True),  # LFM3 SWA ring (window 256, 264 slots) + gate
    (8, 8, 1, 5, 300, 0, 0, False),      # short sequences, MHA
    (16, 2, 1, 4, 900, 0, 0, True),      # two KV heads: one 2-wave workgroup per (sequence, share)
])
def test_dma_plan_head_dim_128(gpu, orc, nq, nkv, n_rows, n_seq, max_ctx, win, cap, gate):
    """Head_dim 128 (two 64-dim halves per row, 16 KB per sub-tile, 2-wave
    workgroups): the forced plan against the oracle and the register plan."""
    la = gpu
    rng = np.random.default_rng(max_ctx + n_seq + nq + win)
    ctx = [int(c) for c in rng.integers(0, max_ctx, size=n_seq)]
    ctx[0] = 0 if not win else 3
    ctx[-1] = max_ctx - 1
    outs = {}
    for plan in ("balanced-dma", "balanced"):
        with la.tuning(plan):
            got, want = _varlen_case(la, orc, np.random.default_rng(11), n_seq, n_rows, nq, nkv, 128, ctx, win=win,
                                     cap=cap, gate=gate, slots=cap or None)
            assert la.last_plan() == plan
        parity(got, want, what=f"{plan} d128 {nq}q/{nkv}kv rows={n_rows} win={win}")
        outs[plan] = got
    assert np.abs(outs["balanced-dma"] - outs["balanced"]).max() < plan_tol(n_rows, nq, nkv)


def test_dma_plan_not_taken_where_ineligible(gpu, orc):
    """Head_dim 128 with two 16-column tiles keeps the register plan under
    the override."""
    la = gpu
    with la.tuning("balanced-dma"):
        got, want = _varlen_case(la, orc, np.random.default_rng(2), 3, 8, 16, 4, 128, [100, 900, 2000])
        assert la.last_plan() == "balanced"
    parity(got, want, what="d128 8 rows under the balanced-dma override")
