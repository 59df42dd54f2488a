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
