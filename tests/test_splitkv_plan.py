"""CPU proof of the balanced split-KV plan's index math (k_splitkv_bal /
k_merge_bal): tests/plan_sim.c runs every workgroup's walk and the merge's slot
range with the kernels' own header (laii_amd/csrc/splitkv_plan.h) and checks
that every attended key of every (sequence, KV head) is covered once
(tools/lfm3_engine.c:862-873 for the row windows), that partial slots are
unique and inside the workspace, and that the merge reads exactly the slots
written.  No GPU needed."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("plan") / "libplansim.so")
    subprocess.run(["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-Werror", "-shared", "-fPIC",
                    "-I", os.path.join(ROOT, "laii_amd", "csrc"), os.path.join(ROOT, "tests", "plan_sim.c"),
                    "-o", out], check=True)
    lib = C.CDLL(out)
    lib.plan_check.restype = C.c_int
    lib.plan_check.argtypes = [C.c_uint32, C.POINTER(C.c_uint32), C.c_uint32, C.c_uint32, C.c_uint32,
                               C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                               C.c_uint32, C.c_int, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                               C.c_char_p, C.c_size_t]

    def check(pos0, n_rows, nkv, W, ncols, window=0, cap=0, n_res=512, target=2048, min_tiles=None,
              keys=None, mutant=0):
        pos0 = np.ascontiguousarray(pos0, np.uint32)
        if min_tiles is None:  # the host's rule (decode_splitkv.hip launch_bal)
            min_tiles = max(2, (12 * ncols + 31) // 32)
        if keys is None:  # the engine's bound: the longest row's keys
            last = pos0.astype(np.int64) + n_rows - 1
            lo = np.maximum(0, last + 1 - window) if window else 0
            keys = int((last - lo + 1).max())
        G, nwg = C.c_uint32(), C.c_uint32()
        msg = C.create_string_buffer(256)
        rc = lib.plan_check(pos0.size, pos0.ctypes.data_as(C.POINTER(C.c_uint32)), n_rows, nkv, W, window, cap,
                            ncols, n_res, target, min_tiles, keys, mutant, C.byref(G), C.byref(nwg), msg, 256)
        return rc, msg.value.decode(), G.value, nwg.value

    return check


def _random_case(rng):
    n_seq = int(rng.integers(1, 131))
    hd = int(rng.choice([64, 128]))
    nkv = int(rng.choice([1, 2, 3, 4, 8]))
    kv_mul = int(rng.choice([1, 2, 4]))
    n_rows = int(rng.choice([1, 1, 1, 2, 8]))
    ncols = n_rows * kv_mul
    if (hd == 64 and ncols > 64) or (hd == 128 and ncols > 32):
        n_rows, ncols = 1, kv_mul
    W = int(rng.choice([1, 2, 4, 8]))
    window = cap = 0
    if rng.random() < 0.25:
        window = int(rng.choice([16, 256]))
        cap = window + int(rng.choice([0, 8])) + (n_rows - 1)
    kind = rng.random()
    if kind < 0.15:  # uniform
        pos0 = np.full(n_seq, int(rng.integers(0, 9000)), np.int64)
    elif kind < 0.3:  # many one-key sequences
        pos0 = np.where(rng.random(n_seq) < 0.5, 0, rng.integers(0, 4000, n_seq))
    else:
        pos0 = rng.integers(0, 9000, n_seq)
    pos0[0] = 0 if rng.random() < 0.5 else pos0[0]
    kw = dict(window=window, cap=cap, n_res=int(rng.choice([64, 256, 512, 1024, 2048])),
              target=int(rng.choice([1024, 2048, 4096])))
    r = rng.random()
    if r < 0.2:  # forced short shares (LFM_ATTN_CHUNK-like): 1-3 tiles per workgroup, no round cap
        kw.update(min_tiles=int(rng.integers(1, 4)), n_res=0x7FFFFFFF, target=0x7FFFFFFF)
    elif r < 0.3:
        kw.update(keys=0)  # no key bound from the caller
    elif r < 0.4:
        kw.update(keys=int(rng.integers(1, 64)))  # a bound that is too small
    return pos0.astype(np.uint32), n_rows, nkv, W, ncols, kw


def test_plan_random_ragged_batches(sim):
    rng = np.random.default_rng(20261202)
    ragged = uniform = 0
    for i in range(2500):
        pos0, n_rows, nkv, W, ncols, kw = _random_case(rng)
        rc, msg, G, nwg = sim(pos0, n_rows, nkv, W, ncols, **kw)
        assert rc == 0, (i, msg, pos0.size, n_rows, nkv, W, ncols, kw)
        assert 1 <= G <= nwg
        if len(set(pos0.tolist())) == 1:
            uniform += 1
        else:
            ragged += 1
    assert ragged > 1000 and uniform > 200


@pytest.mark.parametrize("n_seq,nkv,W,ncols", [(9, 4, 2, 4), (9, 4, 1, 4), (9, 4, 4, 4), (130, 8, 8, 4),
                                               (5, 8, 8, 32), (1, 8, 8, 4), (64, 8, 8, 4)])
def test_plan_gpu_test_batches(sim, n_seq, nkv, W, ncols):
    """The ragged batches the GPU tests run (test_gpu_decode.py::
    test_balanced_plan_matches_grid_plan, seeds and shapes), with every wave
    count the host may pick, and with 96-key shares."""
    hd = 128 if (nkv == 4 and ncols == 4) else 64
    rng = np.random.default_rng(n_seq * 31 + hd)
    ctx = [int(c) for c in rng.integers(0, 3000, size=n_seq)]
    if n_seq > 1:
        ctx[0], ctx[-1] = 0, 2999
    n_rows = ncols // 4 if ncols > 4 else 1
    pos0 = np.asarray(ctx, np.uint32)
    for kw in ({}, dict(min_tiles=3, n_res=0x7FFFFFFF, target=0x7FFFFFFF)):
        rc, msg, _, _ = sim(pos0, n_rows, nkv, W, ncols, **kw)
        assert rc == 0, msg


def test_plan_headline_and_cfg2(sim):
    """Config 2 batches: the north-star (64 x 8192, uniform) and ctx ~ U[512, 8192]."""
    rng = np.random.default_rng(2)
    for pos0 in (np.full(64, 8191, np.uint32), (rng.integers(512, 8193, 64) - 1).astype(np.uint32)):
        for n_res in (256, 512, 768):
            rc, msg, G, _ = sim(pos0, 1, 8, 8, 4, n_res=n_res)
            assert rc == 0, msg


@pytest.mark.parametrize("mutant", [1, 2, 3])
def test_plan_check_rejects_planted_mistakes(sim, mutant):
    """The checks have teeth: each planted index mistake is rejected on some
    of the batches above."""
    rng = np.random.default_rng(5)
    caught = 0
    for _ in range(200):
        pos0, n_rows, nkv, W, ncols, kw = _random_case(rng)
        rc, _, _, _ = sim(pos0, n_rows, nkv, W, ncols, mutant=mutant, **kw)
        caught += rc != 0
    assert caught > 20, caught


# ---- plan choice of the launch path (host only: lfm_attn_plan_preview) -------------------------

BASELINE_PLANS = [
    # (name, preview kwargs, expected (plan, waves))
    ("cfg1 decode B1 16q/8kv ctx 1024", dict(n_seq=1, n_rows=1, n_head_q=16, n_head_kv=8, head_dim=64,
                                            keys_hint=1024, positions_on_device=False), ("grid", 1)),
    ("cfg1 engine step (fused)", dict(n_seq=1, n_rows=1, n_head_q=16, n_head_kv=8, head_dim=64, keys_hint=1024,
                                      fused=True), ("grid", 1)),
    ("cfg2 B64 x 8192", dict(n_seq=64, n_rows=1, n_head_q=32, n_head_kv=8, head_dim=64, keys_hint=8192),
     ("balanced", 8)),
    ("cfg2 fused step", dict(n_seq=64, n_rows=1, n_head_q=32, n_head_kv=8, head_dim=64, keys_hint=8192,
                             fused=True), ("balanced", 8)),
    ("cfg3 verify B16 x 8 rows", dict(n_seq=16, n_rows=8, n_head_q=32, n_head_kv=8, head_dim=64, keys_hint=4104),
     ("balanced-dma", 4)),
    ("cfg3 fused verify step", dict(n_seq=16, n_rows=8, n_head_q=32, n_head_kv=8, head_dim=64, keys_hint=4104,
                                    fused=True), ("balanced", 8)),
    ("cfg5 SWA ring", dict(n_seq=32, n_rows=1, n_head_q=16, n_head_kv=4, head_dim=128, window_len=256,
                           keys_hint=256), ("wg", 4)),
    ("cfg5 full B32 x 32768", dict(n_seq=32, n_rows=1, n_head_q=16, n_head_kv=4, head_dim=128, keys_hint=32768),
     ("balanced", 2)),
]


@pytest.mark.parametrize("name,kw,want", BASELINE_PLANS, ids=[c[0] for c in BASELINE_PLANS])
def test_plan_choice_baseline_shapes(name, kw, want):
    """The launch form each BASELINE configuration takes on a 256-CU MI355X
    (the forms the bench measures), computed on the host without a device."""
    import laii_amd as la
    plan, waves, splits, chunk = la.plan_preview(**kw)
    assert (plan, waves) == want, (name, plan, waves)
    if not plan.startswith("balanced"):
        keys = kw["keys_hint"]
        assert splits >= 1 and chunk % 32 == 0 and splits * chunk >= min(keys, kw.get("window_len") or keys)


def test_plan_overrides_and_lds_budget():
    """Overrides force a form and counts, and clear back to the automatic
    choice; a forced in-workgroup form whose fused LDS (V tiles + staged new
    rows) would pass 64 KB falls back to the grid, with fewer waves."""
    import laii_amd as la
    cfg2 = dict(n_seq=64, n_rows=1, n_head_q=32, n_head_kv=8, head_dim=64, keys_hint=8192)
    with la.tuning("grid", chunk=96):
        assert la.plan_preview(**cfg2)[0] == "grid" and la.plan_preview(**cfg2)[3] == 96
    with la.tuning("wg"):
        assert la.plan_preview(**cfg2)[0] == "wg"
        mha = dict(n_seq=1, n_rows=64, n_head_q=8, n_head_kv=8, head_dim=64, keys_hint=4096, fused=True)
        plan, waves, _, _ = la.plan_preview(**mha)
        assert plan == "grid" and waves <= 2, (plan, waves)
    with la.tuning(waves=2):
        assert la.plan_preview(**cfg2)[:2] == ("balanced", 2)
    assert la.plan_preview(**cfg2)[:2] == ("balanced", 8)
    # the LDS-streamed form: head_dim 64, at most 32 query columns, no fused
    # prologue; forced or (two 16-column tiles) by default
    verify = dict(n_seq=16, n_rows=8, n_head_q=32, n_head_kv=8, head_dim=64, keys_hint=4104)
    with la.tuning("balanced-dma"):
        assert la.plan_preview(**cfg2)[:2] == ("balanced-dma", 4)
        assert la.plan_preview(**dict(cfg2, fused=True))[:2] == ("balanced", 8)
        assert la.plan_preview(**dict(cfg2, head_dim=128, n_head_q=16, n_head_kv=4))[:2] == ("balanced-dma", 2)
        assert la.plan_preview(**dict(cfg2, head_dim=128, n_head_q=16, n_head_kv=4, n_rows=8))[0] == "balanced"
        assert la.plan_preview(**dict(verify, n_rows=16))[0] == "balanced"  # 64 columns
    with la.tuning("balanced"):
        assert la.plan_preview(**verify)[:2] == ("balanced", 8)
    with la.tuning(waves=8):
        assert la.plan_preview(**verify)[:2] == ("balanced", 8)
    with pytest.raises(la.LfmAttnError):
        la.set_tuning("fastest")
    with pytest.raises(la.LfmAttnError):
        la.set_tuning(waves=3)
    assert la.plan_preview(n_seq=1, n_rows=1, n_head_q=4, n_head_kv=2, head_dim=32)[0] == "generic"
