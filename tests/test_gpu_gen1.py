"""GPU parity of the Gen-1 FP32 attention step (lfm_hip_gen1_gqa_step),
steps 2-4 of lfm_gqa_step (src/lfm_forward.c:184-244): QK-RMSNorm, per-call
NeoX RoPE, FP32 KV append and softmax attention."""
import os
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def _run(la, q, k, v, qn, kn, kc, vc, pos, nq, nkv, hd, eps=1e-5, theta=1e6):
    """Upload, run the step on the device, return attn_out and the caches."""
    c, s = la.rope_row_gen1(hd, pos, theta)
    kd, vd = dev(la, kc), dev(la, vc)
    out = la.DeviceArray.zeros(nq * hd, np.float32)
    la.gen1_gqa_step(dev(la, q), dev(la, k), dev(la, v), None if qn is None else dev(la, qn),
                     None if kn is None else dev(la, kn), kd, vd, out, pos, kc.shape[0], nq, nkv, hd, eps,
                     dev(la, c), dev(la, s))
    return out.numpy(), kd.numpy(), vd.numpy()


def test_gen1_fixture_on_gpu(gpu):
    """tests/fixtures_attention.bin (the reference's PyTorch fixture,
    tools/generate_reference_tensors.py:77-164): D 64, 4q/2kv, d16, pos 5.
    Projections and wo in float64 on the host; the reference's own gate is
    1e-4 (tests/test_attention.c:105)."""
    la = gpu
    raw = open(os.path.join(GOLDEN, "fixtures_attention.bin"), "rb").read()
    D, nq, nkv, hd, pos, _ = struct.unpack("6I", raw[:24])
    f = np.frombuffer(raw[24:], np.float32)
    o = 0

    def take(n, shape):
        nonlocal o
        a = f[o:o + n].reshape(shape)
        o += n
        return a

    x = take(D, (D,))
    wq, wk, wv = take(nq * hd * D, (nq * hd, D)), take(nkv * hd * D, (nkv * hd, D)), take(nkv * hd * D, (nkv * hd, D))
    qn, kn = take(hd, (hd,)), take(hd, (hd,))
    wo = take(D * D, (D, D))
    kh, vh = take(pos * nkv * hd, (pos, nkv * hd)), take(pos * nkv * hd, (pos, nkv * hd))
    expected = take(D, (D,))
    q = (wq.astype(np.float64) @ x).astype(np.float32)
    k = (wk.astype(np.float64) @ x).astype(np.float32)
    v = (wv.astype(np.float64) @ x).astype(np.float32)
    kc = np.zeros((pos + 10, nkv * hd), np.float32)
    vc = np.zeros((pos + 10, nkv * hd), np.float32)
    kc[:pos], vc[:pos] = kh, vh
    att, _, gv = _run(la, q, k, v, qn, kn, kc, vc, pos, nq, nkv, hd)
    out = wo.astype(np.float64) @ att
    err = float(np.abs(out - expected).max())
    print(f"gen1 fixture: max_abs={err:.3e}")
    assert err < 1e-4
    assert np.array_equal(gv[pos], v)


@pytest.mark.parametrize("nq,nkv,hd,pos,norm", [(32, 8, 64, 300, True), (16, 4, 128, 77, True),
                                                (4, 2, 16, 5, True), (8, 8, 40, 0, True), (12, 4, 96, 1000, False)])
def test_gen1_vs_oracle(gpu, orc, nq, nkv, hd, pos, norm):
    """Against the oracle's Gen-1 step, which is bit-identical to the
    reference's lfm_gqa_step (tests/test_oracle.py): the appended K row bit for
    bit (same sum-of-squares order, libm angles, separately rounded rotation),
    V copied, attention within 2e-6 (the GPU adds the softmax in another
    order)."""
    la = gpu
    rng = np.random.default_rng(pos + hd)
    q = rng.standard_normal(nq * hd).astype(np.float32) * 2
    k = rng.standard_normal(nkv * hd).astype(np.float32) * 2
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32) if norm else None
    kc = rng.standard_normal((pos + 3, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((pos + 3, nkv * hd)).astype(np.float32)
    att, gk, gv = _run(la, q, k, v, qn, kn, kc, vc, pos, nq, nkv, hd)
    kc2, vc2 = kc.copy(), vc.copy()
    want = orc.gen1_gqa_attend(q, k, v, qn, kn, kc2, vc2, pos, nq, nkv, hd, 1e-5, 1e6)
    assert np.array_equal(gk, kc2), "K cache (appended row) differs"
    assert np.array_equal(gv, vc2)
    err = float(np.abs(att - want).max())
    print(f"gen1 {nq}q/{nkv}kv d{hd} pos {pos}: max_abs={err:.3e}")
    assert err < 2e-6
