"""Launch shape of the head_dim-128/64 prefill (lfm_hip_lfm3_prefill_f16),
computed on the host (lfm_attn_prefill_plan_preview): tile size, tiles per
workgroup, the short tiles at the sequence start that a sliding-window launch
dispatches first, workgroups.  No GPU needed.

The short tiles are checked against the window's own definition: row at
position p attends keys [p + 1 - window, p] (tools/lfm3_engine.c:862-873),
so a tile is short exactly when its first row's window starts before
position 0."""
import numpy as np
import pytest

import laii_amd as la


def preview(**kw):
    return la.prefill_plan_preview(**kw)


def test_bench_window_shape():
    """The bench's sliding-window row: B4 x 4096, 16q/4kv, window 256."""
    tq, chain, n_light, n_wg = preview(n_seq=4, n_tok=4096, n_head_q=16, n_head_kv=4, head_dim=128,
                                       window_len=256)
    assert (tq, chain, n_wg) == (32, 1, 128 * 4 * 4)
    assert n_light == 8  # positions 0..255: tiles 0..7


def test_full_layer_keeps_heaviest_first():
    tq, chain, n_light, n_wg = preview(n_seq=4, n_tok=4096, n_head_q=16, n_head_kv=4, head_dim=128)
    assert (tq, chain, n_light, n_wg) == (32, 1, 0, 128 * 16)


@pytest.mark.parametrize("seed", range(6))
def test_short_tiles_match_the_window_definition(seed):
    """For random prompts, the tiles dispatched first are exactly the
    leading tiles whose first row's window reaches before position 0."""
    rng = np.random.default_rng(seed)
    for _ in range(200):
        nkv = int(rng.choice([1, 2, 4, 8, 16]))
        nq = nkv * int(rng.choice([1, 2, 4, 8]))
        n_tok = int(rng.integers(1, 3000))
        pos_0 = int(rng.choice([0, 0, int(rng.integers(0, 2000))]))
        window = int(rng.choice([0, 1, 33, 200, 256, 512, 4096]))
        tq, chain, n_light, n_wg = preview(n_seq=2, n_tok=n_tok, n_head_q=nq, n_head_kv=nkv, head_dim=128,
                                           pos_0=pos_0, window_len=window)
        assert tq == 128 // (nq // nkv)
        n_qtiles = -(-n_tok // tq)
        assert chain == 1 and n_wg == n_qtiles * nkv * 2
        short = [i for i in range(n_qtiles) if window and pos_0 + i * tq + 1 < window]
        assert short == list(range(n_light)), (n_tok, pos_0, window, tq, n_light)


def test_forced_chain_disables_the_short_first_order():
    with la.tuning(prefill_chain=3):
        tq, chain, n_light, n_wg = preview(n_seq=1, n_tok=700, n_head_q=16, n_head_kv=4, head_dim=128,
                                           window_len=256)
    assert (tq, chain, n_light) == (32, 3, 0)
    assert n_wg == -(-22 // 3) * 4
    # a full layer ignores the override
    with la.tuning(prefill_chain=3):
        assert preview(n_seq=1, n_tok=700, n_head_q=16, n_head_kv=4, head_dim=128)[1] == 1


def test_rejects_shapes_the_entry_point_does_not_take():
    with pytest.raises(la.LfmAttnError):
        preview(n_seq=1, n_tok=64, n_head_q=16, n_head_kv=4, head_dim=96)
    with pytest.raises(la.LfmAttnError):
        preview(n_seq=1, n_tok=64, n_head_q=15, n_head_kv=4, head_dim=128)
    with pytest.raises(la.LfmAttnError):
        preview(n_seq=0, n_tok=64, n_head_q=16, n_head_kv=4, head_dim=128)
