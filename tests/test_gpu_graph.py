"""The allocation-free decode entry point (lfm_hip_gqa_f16_varlen_noalloc)
captured into a HIP graph on a caller stream -- the use it exists for: the
call allocates nothing and records no memset, only kernel launches.  Each
graph is replayed several times, with the program's own eager calls and
synchronizations between the replays, and every replay must equal the eager
call bit for bit.  One case per plan: the two-kernel grid (one sequence),
the balanced plan with its merge (a ragged batch), and the in-workgroup
merge (an LFM3 sliding-window ring with a gate)."""
import ctypes as C
import os

import numpy as np
import pytest

from helpers import rand_kv

pytestmark = pytest.mark.gpu


class HipGraphs:
    """The few HIP runtime calls of stream capture (plumbing only)."""

    def __init__(self):
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        self.lib = C.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
        L = self.lib
        for n, args in (("hipStreamCreate", [C.POINTER(C.c_void_p)]),
                        ("hipStreamDestroy", [C.c_void_p]),
                        ("hipStreamSynchronize", [C.c_void_p]),
                        ("hipStreamBeginCapture", [C.c_void_p, C.c_int]),
                        ("hipStreamEndCapture", [C.c_void_p, C.POINTER(C.c_void_p)]),
                        ("hipGraphInstantiate", [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p,
                                                 C.c_size_t]),
                        ("hipGraphLaunch", [C.c_void_p, C.c_void_p]),
                        ("hipGraphExecDestroy", [C.c_void_p]),
                        ("hipGraphDestroy", [C.c_void_p])):
            getattr(L, n).restype = C.c_int
            getattr(L, n).argtypes = args

    def stream(self):
        s = C.c_void_p()
        assert self.lib.hipStreamCreate(C.byref(s)) == 0
        return s

    def capture(self, stream, fn):
        """fn() enqueues on stream; returns (graph, exec)."""
        assert self.lib.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
        err = None
        try:
            fn()
        except Exception as e:  # end the capture before reporting
            err = e
        g = C.c_void_p()
        rc = self.lib.hipStreamEndCapture(stream, C.byref(g))
        if err is not None:
            raise err
        assert rc == 0, f"hipStreamEndCapture: {rc}"
        x = C.c_void_p()
        assert self.lib.hipGraphInstantiate(C.byref(x), g, None, None, 0) == 0
        return g, x


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def _batch(la, rng, n_seq, n_rows, nq, nkv, hd, ctx, win=0, cap=0, gate=False):
    pos0 = np.asarray(ctx, np.uint32)
    kd, vd = [], []
    for s in range(n_seq):
        n_slots = cap if cap else int(pos0[s]) + n_rows
        kd.append(dev(la, rand_kv(rng, n_slots, nkv, hd)))
        vd.append(dev(la, rand_kv(rng, n_slots, nkv, hd)))
    q = rng.standard_normal((n_seq, n_rows, nq, hd), dtype=np.float32)
    g = rng.standard_normal((n_seq, n_rows, nq)).astype(np.float32) if gate else None
    keys = int(win + n_rows - 1) if win else int(pos0.max() + n_rows)
    args = (dev(la, q), None if g is None else dev(la, g), True, la.pointer_table(kd), la.pointer_table(vd),
            dev(la, pos0))
    tail = (n_seq, n_rows, keys, nq, nkv, hd, win, cap)
    return args, tail, q.shape, (kd, vd)


@pytest.mark.parametrize("name,shape", [
    ("grid, one sequence", dict(n_seq=1, n_rows=1, nq=16, nkv=8, hd=64, ctx=[1023])),
    ("balanced, ragged", dict(n_seq=8, n_rows=1, nq=32, nkv=8, hd=64, ctx=[5, 700, 4096, 33, 1500, 2047, 1, 900])),
    ("balanced LDS-streamed, verify rows", dict(n_seq=6, n_rows=8, nq=32, nkv=8, hd=64,
                                                ctx=[4096, 17, 2500, 900, 4096, 64])),
    ("in-workgroup merge, ring + gate", dict(n_seq=4, n_rows=1, nq=16, nkv=4, hd=128, ctx=[1000] * 4,
                                             win=256, cap=264, gate=True)),
])
def test_noalloc_graph_replays_match_eager(gpu, name, shape):
    la = gpu
    hg = HipGraphs()
    rng = np.random.default_rng(4242)
    args, tail, oshape, keep = _batch(la, rng, **shape)
    stream = hg.stream()
    try:
        eager = la.DeviceArray.zeros(oshape, np.float32)
        la.gqa_f16_varlen_noalloc(*args, eager, *tail, stream=stream)
        assert hg.lib.hipStreamSynchronize(stream) == 0
        want = eager.numpy()
        plan = la.last_plan()

        replay = la.DeviceArray.zeros(oshape, np.float32)
        graph, gexec = hg.capture(stream, lambda: la.gqa_f16_varlen_noalloc(*args, replay, *tail, stream=stream))
        try:
            other = la.DeviceArray.zeros(oshape, np.float32)
            for rep in range(4):
                replay.upload(np.zeros(oshape, np.float32))  # synchronous, outside the graph
                assert hg.lib.hipGraphLaunch(gexec, stream) == 0
                assert hg.lib.hipStreamSynchronize(stream) == 0
                got = replay.numpy()
                assert np.array_equal(got, want), f"{name} ({plan}): replay {rep} differs from the eager call"
                # the program's own eager work between replays, on the same
                # stream and the same fixed partial array
                la.gqa_f16_varlen_noalloc(*args, other, *tail, stream=stream)
                assert hg.lib.hipStreamSynchronize(stream) == 0
                assert np.array_equal(other.numpy(), want), f"{name}: eager call {rep} differs"
        finally:
            hg.lib.hipGraphExecDestroy(gexec)
            hg.lib.hipGraphDestroy(graph)
    finally:
        hg.lib.hipStreamSynchronize(stream)
        hg.lib.hipStreamDestroy(stream)
