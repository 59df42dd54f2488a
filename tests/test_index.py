"""Positions, windows and ring slots: bit-exact, exhaustively.

The product maps an attended absolute position p to slot p % cap (window) or
p (linear); the reference walks seg1 from t_start % cap then seg2 from slot 0
(tools/lfm3_engine.c:862-873, 1103-1114).  Both are checked against a brute
force enumeration of the window, for every position in [0, 4*cap)."""
import numpy as np
import pytest

import laii_amd as la


def brute_window(abs_pos, window):
    lo = 0 if window == 0 else max(0, abs_pos + 1 - window)
    return list(range(lo, abs_pos + 1))


@pytest.mark.parametrize("cap,window", [(24, 16), (24, 24), (256, 256), (264, 256), (5, 5),
                                        (17, 9), (32, 32), (33, 31), (264, 1)])
def test_ring_plan_exhaustive(orc, cap, window):
    for abs_pos in range(4 * cap):
        plan = la.seg_plan(abs_pos, window, cap)
        assert plan == orc.lfm3_plan(abs_pos, window, cap)
        t_start, count, seg1_slot, seg1_len, seg2_len = plan
        positions = brute_window(abs_pos, window)
        assert t_start == positions[0] and count == len(positions)
        walk = orc.lfm3_slots(abs_pos, window, cap)
        mapped = [la.slot_of(p, window, cap) for p in positions]
        assert list(walk) == mapped
        assert mapped == [p % cap for p in positions]
        assert len(set(mapped)) == len(mapped)  # window fits the ring: no slot twice
        assert seg1_len + seg2_len == count and seg1_slot + seg1_len <= cap


def test_linear_plan(orc):
    for abs_pos in list(range(200)) + [4095, 8191, 32767]:
        plan = la.seg_plan(abs_pos, 0, 0)
        assert plan == (0, abs_pos + 1, 0, abs_pos + 1, 0)
        assert plan == orc.lfm3_plan(abs_pos, 0, 1 << 20)
        assert la.slot_of(abs_pos, 0, 0) == abs_pos


def test_ring_special_cases():
    """pos 1000, window 256: cap 256 -> slots 233..255 then 0..232;
    cap 264 -> slots 217..263 then 0..208."""
    assert la.seg_plan(1000, 256, 256) == (745, 256, 233, 23, 233)
    assert la.seg_plan(1000, 256, 264) == (745, 256, 217, 47, 209)
    # segment boundary exactly at cap: t_start % cap == 0 -> one segment
    assert la.seg_plan(263 + 264, 264, 264) == (264, 264, 0, 264, 0)
    # before the window fills: no wrap, starts at 0
    assert la.seg_plan(100, 256, 264) == (0, 101, 0, 101, 0)


def test_batched_rows_causal_bounds():
    """Row b of a B-row batch is position pos_0 + b (tools/lfm3_engine.c:863-869):
    its window never reaches a later row's position."""
    for pos_0 in (0, 7, 250, 1000):
        for b in range(8):
            t0, count, *_ = la.seg_plan(pos_0 + b, 256, 264)
            assert t0 + count - 1 == pos_0 + b
    rng = np.random.default_rng(0)
    for _ in range(2000):
        cap = int(rng.integers(1, 600))
        window = int(rng.integers(1, cap + 1))
        p = int(rng.integers(0, 1 << 31))
        plan = la.seg_plan(p, window, cap)
        assert plan[0] == max(0, p + 1 - window) and plan[2] == plan[0] % cap
