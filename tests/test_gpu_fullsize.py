"""GPU parity at the BASELINE configurations' full sizes, against the CPU
oracle (the restatement of the reference workers), through the C-ABI.

  cfg2  B64 decode, 32q/8kv d64, ctx ~ U[512, 8192] and the all-8192
        north-star batch; the new token's raw q/k/v go through the QK-RMSNorm
        + RoPE (theta 1e6) prologue, then the attention
        (tools/lfm2_kernels_fast.c:403-497, 700-810, 1046-1066)
  cfg3  speculative verify, B16 x 8 causal rows over ctx 4096 + 8
        (tools/lfm2_speculative_pld.c:388-461)
  cfg5  LFM3 full layer, B32 x ctx 32768, 16q/4kv d128, partial RoPE
        (rope_freqs 1 x 32, 1e30 x 32), sigmoid gate
        (tools/lfm3_engine.c:403-450, 851-946, 1588-1597)

K/V caches are 0.5 * N(0,1) rounded to fp16 and queries N(0,1), as BASELINE
draws them.

Every sequence is also checked by properties that hold at any size: finite
outputs, and each output dim inside [min, max] of that dim over the values
the row attends (a softmax is a convex combination)."""
import os

import numpy as np
import pytest

from helpers import f16, f16_to_f32, parity

pytestmark = pytest.mark.gpu

EPS = 1e-5


def dev(la, arr):
    return la.DeviceArray.from_numpy(np.ascontiguousarray(arr))


def normal_kv(seed, slots, nkv, hd):
    """fp16 cache rows of 0.5 * N(0,1), BASELINE's K/V distribution: one
    seeded float32 draw per sequence (child streams of SeedSequence(seed)),
    rounded to nearest even, drawn on threads (gigabytes at full size)."""
    from concurrent.futures import ThreadPoolExecutor

    def one(args):
        child, n = args
        x = np.random.default_rng(child).standard_normal((n, nkv, hd), dtype=np.float32)
        x *= np.float32(0.5)
        return x.astype(np.float16).view(np.uint16)

    kids = np.random.SeedSequence(seed).spawn(len(slots))
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        return list(ex.map(one, zip(kids, [int(n) for n in slots])))


def check_convex(out, lo, hi, what):
    tol = 1e-5 * np.maximum(1.0, np.abs(hi))
    assert np.all(np.isfinite(out)), f"{what}: non-finite"
    assert np.all(out >= lo - tol) and np.all(out <= hi + tol), f"{what}: outside the convex hull"


class _Decode:
    """n_seq sequences; the last position of sequence s is ctx[s] - 1.  The
    caches hold random rows at positions 0 .. ctx[s] - 2; the new token's
    row at ctx[s] - 1 is written by the prologue from raw k/v."""

    def __init__(self, la, rng, ctx, nq, nkv, hd, cos, sin, orc_lut, gate=False):
        self.la, self.nq, self.nkv, self.hd = la, nq, nkv, hd
        self.ctx = np.asarray(ctx, np.int64)
        self.n_seq = len(ctx)
        self.pos = (self.ctx - 1).astype(np.uint32)
        seed = int(rng.integers(1 << 31))
        self.k = normal_kv(seed, self.ctx, nkv, hd)
        self.v = normal_kv(seed + 1, self.ctx, nkv, hd)
        self.kd = [dev(la, k) for k in self.k]
        self.vd = [dev(la, v) for v in self.v]
        self.kt, self.vt = la.pointer_table(self.kd), la.pointer_table(self.vd)
        self.q_raw = rng.standard_normal((self.n_seq, nq, hd), dtype=np.float32)
        self.k_raw = rng.standard_normal((self.n_seq, nkv, hd), dtype=np.float32)
        self.v_raw = rng.standard_normal((self.n_seq, nkv, hd), dtype=np.float32)
        self.qw = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        self.kw = (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32)
        self.g = rng.standard_normal((self.n_seq, nq)).astype(np.float32) if gate else None
        self.cos, self.sin = orc_lut  # the oracle's own tables for the oracle side
        self.cd, self.sd = dev(la, cos), dev(la, sin)

    def run_two_launch(self):
        """lfm_hip_qkv_prologue, then lfm_hip_gqa_f16_varlen."""
        la = self.la
        qd = dev(la, self.q_raw)
        out = la.DeviceArray.zeros(self.q_raw.shape, np.float32)
        posd = dev(la, self.pos)
        la.qkv_prologue(qd, dev(la, self.k_raw), dev(la, self.v_raw), self.kt, self.vt, posd, self.n_seq, 1,
                        self.nq, self.nkv, self.hd, dev(la, self.qw), dev(la, self.kw), EPS, self.cd, self.sd)
        la.gqa_f16_varlen(qd, None if self.g is None else dev(la, self.g), True, self.kt, self.vt, posd, out,
                          self.n_seq, 1, int(self.ctx.max()), self.nq, self.nkv, self.hd)
        return out.numpy()

    def run_fused(self):
        """lfm_hip_gqa_f16_step: the prologue inside the attention kernel."""
        la = self.la
        out = la.DeviceArray.zeros(self.q_raw.shape, np.float32)
        qd = dev(la, self.q_raw)
        la.gqa_f16_step(qd, dev(la, self.k_raw), dev(la, self.v_raw), None if self.g is None else dev(la, self.g),
                        True, self.kt, self.vt, dev(la, self.pos), out, self.n_seq, 1, int(self.ctx.max()), self.nq,
                        self.nkv, self.hd, dev(la, self.qw), dev(la, self.kw), EPS, self.cd, self.sd)
        assert np.array_equal(qd.numpy(), self.q_raw)
        return out.numpy()

    def run(self, mode):
        return self.run_fused() if mode == "fused" else self.run_two_launch()

    def caches_after(self, s):
        """The device caches of sequence s (with the prologue's new row)."""
        return self.kd[s].numpy(), self.vd[s].numpy()

    def oracle(self, orc, s, k16, v16):
        p = int(self.pos[s])
        q = orc.qk_norm_rope(self.q_raw[s], self.nq, self.hd, self.qw, EPS, self.cos[p], self.sin[p])
        want_k = orc.qk_norm_rope(self.k_raw[s], self.nkv, self.hd, self.kw, EPS, self.cos[p], self.sin[p],
                                  store_f16=True)
        assert np.array_equal(k16[p].reshape(-1), want_k), f"seq {s}: new K row"
        assert np.array_equal(v16[p].reshape(-1), f16(self.v_raw[s]).reshape(-1)), f"seq {s}: new V row"
        g = None if self.g is None else (1.0 / (1.0 + np.exp(-self.g[s]))).astype(np.float32)
        return orc.lfm3_online_gqa_f16(q, g, k16, v16, 1, p, 0, p + 1, self.nq, self.nkv, self.hd)

    def check(self, orc, got, sample, what):
        kv_mul = self.nq // self.nkv
        for s in range(self.n_seq):
            k16, v16 = self.caches_after(s)
            p = int(self.pos[s])
            o = got[s].reshape(self.nq, self.hd)
            vf = f16_to_f32(v16[:p + 1])
            vlo, vhi = vf.min(axis=0), vf.max(axis=0)  # [nkv][hd]
            for h in range(self.nq):
                lo, hi = vlo[h // kv_mul], vhi[h // kv_mul]
                if self.g is None:
                    check_convex(o[h], lo, hi, f"{what} seq {s} head {h}")
                else:
                    gs = 1.0 / (1.0 + np.exp(-np.float64(self.g[s, h])))
                    check_convex(o[h] / gs, lo, hi, f"{what} seq {s} head {h}")
            if s in sample:
                parity(got[s], self.oracle(orc, s, k16, v16), what=f"{what} seq {s} ctx {p + 1}")


@pytest.mark.parametrize("mode", ["two_launch", "fused"])
@pytest.mark.parametrize("kind", ["ragged", "northstar"])
def test_cfg2_fullsize_prologue_then_decode(gpu, orc, kind, mode):
    """Config 2: 64 sequences, 32q/8kv d64, ctx ~ U[512, 8192] (and all 8192),
    QK-RMSNorm (w = 1 + 0.05 N, eps 1e-5) + RoPE theta 1e6 of the new token,
    then batched decode -- as two launches (lfm_hip_qkv_prologue, then
    lfm_hip_gqa_f16_varlen) and fused (lfm_hip_gqa_f16_step).  Every sequence
    against the oracle and by bounds."""
    la = gpu
    rng = np.random.default_rng(2 if kind == "ragged" else 8192)
    ctx = rng.integers(512, 8193, size=64) if kind == "ragged" else np.full(64, 8192)
    if kind == "ragged":
        ctx[0], ctx[1] = 512, 8192
    cos, sin = la.rope_lut_lfm2(8192, 64, 1e6)
    d = _Decode(la, rng, ctx, 32, 8, 64, cos, sin, orc.rope_lut_lfm2(8192, 64, 1e6))
    got = d.run(mode)
    d.check(orc, got, set(range(64)), f"cfg2 {kind} {mode}")


def test_cfg3_fullsize_verify(gpu, orc):
    """Config 3: 16 sequences x 8 causal rows at positions 4096 .. 4103 (row
    r attends 4097 + r keys), 32q/8kv d64; every sequence against the oracle."""
    la = gpu
    rng = np.random.default_rng(3)
    n_seq, n_rows, nq, nkv, hd = 16, 8, 32, 8, 64
    pos0 = np.full(n_seq, 4096, np.uint32)
    k = normal_kv(31, [4104] * n_seq, nkv, hd)
    v = normal_kv(32, [4104] * n_seq, nkv, hd)
    kd, vd = [dev(la, x) for x in k], [dev(la, x) for x in v]
    q = rng.standard_normal((n_seq, n_rows, nq, hd), dtype=np.float32)
    out = la.DeviceArray.zeros(q.shape, np.float32)
    la.gqa_f16_varlen(dev(la, q), None, True, la.pointer_table(kd), la.pointer_table(vd), dev(la, pos0), out,
                      n_seq, n_rows, 4104, nq, nkv, hd)
    got = out.numpy()
    for s in range(n_seq):
        want = orc.lfm3_online_gqa_f16(q[s], None, k[s], v[s], n_rows, 4096, 0, 4104, nq, nkv, hd)
        parity(got[s], want, what=f"cfg3 seq {s}")
        vf = f16_to_f32(v[s])
        for r in range(n_rows):
            vlo, vhi = vf[:4097 + r].min(axis=0), vf[:4097 + r].max(axis=0)
            for h in range(nq):
                check_convex(got[s, r, h], vlo[h // 4], vhi[h // 4], f"cfg3 seq {s} row {r} head {h}")


@pytest.mark.parametrize("mode", ["two_launch", "fused"])
def test_cfg5_fullsize_lfm3_full_layer(gpu, orc, mode):
    """Config 5, full-attention layer: 32 sequences x ctx 32768, 16q/4kv
    d128, partial-RoPE prologue (theta 1e6; pairs i < 32 rotate, the rest are
    identity) and the sigmoid gate from logits.  16 sequences against the
    oracle, all 32 by bounds."""
    la = gpu
    rng = np.random.default_rng(5)
    rf = np.array([1.0] * 32 + [1e30] * 32, np.float32)
    cos, sin = la.rope_lut_lfm3(32768, 128, 128, 1e6, rf)
    d = _Decode(la, rng, np.full(32, 32768), 16, 4, 128, cos, sin, orc.rope_lut_lfm3(32768, 128, 128, 1e6, rf),
                gate=True)
    got = d.run(mode)
    d.check(orc, got, set(range(0, 32, 2)) | {31}, f"cfg5 full {mode}")
