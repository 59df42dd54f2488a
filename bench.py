#!/usr/bin/env python3
"""Benchmark of the MI355X attention path (one GPU).

Headline (value): batched decode attention, LFM2-1.2B GQA shape -- 64
independent sequences, 32 query / 8 KV heads, head_dim 64, fp16 KV, every
context 8192 (north-star size).  One step = one attention
call over the whole batch (split-KV kernel + merge), inputs resident in HBM.
value = algorithmic bytes / step time (KV read once + Q read + O written).

Also reported: config 2 with ctx ~ U[512, 8192], config 3 (B=8 speculative
verify), config 5 (LFM3 SWA ring and full layer), each as GB/s, and the
reference's CPU attention timed on this host (cpu_baseline).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, datasheet
# HBM bytes per launch of the headline kernel from two rocprofv3 PMC passes
# (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000, factors from a 2 GiB read/copy
# kernel); profiles/k_splitkv_decode_b64_ctx8192_pmc.md
HEADLINE_TRAFFIC_BYTES = 1078550016
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense fp16 MFMA, datasheet


class Hip:
    """Minimal HIP runtime access for events (plumbing only)."""

    def __init__(self):
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        self.lib = C.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
        for n in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize",
                  "hipEventElapsedTime", "hipDeviceSynchronize", "hipEventDestroy"):
            getattr(self.lib, n).restype = C.c_int
        self.lib.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.lib.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [C.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.lib.hipEventDestroy.argtypes = [C.c_void_p]

    def event(self):
        ev = C.c_void_p()
        assert self.lib.hipEventCreate(C.byref(ev)) == 0
        return ev

    def record(self, ev, stream=None):
        assert self.lib.hipEventRecord(ev, stream) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.lib.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.lib.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return float(ms.value)

    def sync(self):
        assert self.lib.hipDeviceSynchronize() == 0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


class DecodeWorkload:
    """n_seq sequences, n_rows query rows each (row r at position pos0[s] + r),
    `copies` independent replicas of all device inputs (rotated per step so
    the working set exceeds the 256 MB last-level cache)."""

    def __init__(self, la, rng, name, n_seq, n_rows, nq, nkv, hd, ctx, window=0, cap=0,
                 gate=False, copies=1, keep_host=0):
        self.la, self.name = la, name
        self.n_seq, self.n_rows, self.nq, self.nkv, self.hd = n_seq, n_rows, nq, nkv, hd
        self.window, self.cap = window, cap
        ctx = np.asarray(ctx, np.int64)
        self.pos0 = (ctx if n_rows > 1 else ctx - 1).astype(np.uint32)  # first row position
        last = self.pos0.astype(np.int64) + n_rows - 1
        self.slots = [int(cap) if window else int(l) + 1 for l in last]
        if window:
            t0 = np.maximum(0, last + 1 - window)
            self.keys = (last - t0 + 1).astype(np.int64)
        else:
            self.keys = last + 1
        self.keys_hint = int(self.keys.max())  # upper bound of keys per row (sizes the grid)
        self.host_k, self.host_v = [], []
        self.sets = []
        for c in range(copies):
            kd, vd = [], []
            for s in range(n_seq):
                k = f16(rng.standard_normal((self.slots[s], nkv, hd), dtype=np.float32) * np.float32(0.5))
                v = f16(rng.standard_normal((self.slots[s], nkv, hd), dtype=np.float32) * np.float32(0.5))
                if c == 0 and s < keep_host:
                    self.host_k.append(k)
                    self.host_v.append(v)
                kd.append(la.DeviceArray.from_numpy(k))
                vd.append(la.DeviceArray.from_numpy(v))
            q = rng.standard_normal((n_seq, n_rows, nq, hd), dtype=np.float32)
            g = rng.standard_normal((n_seq, n_rows, nq)).astype(np.float32) if gate else None
            if c == 0:
                self.host_q, self.host_g = q, g
            self.sets.append(dict(kd=kd, vd=vd, kt=la.pointer_table(kd), vt=la.pointer_table(vd),
                                  q=la.DeviceArray.from_numpy(q),
                                  g=None if g is None else la.DeviceArray.from_numpy(g),
                                  out=la.DeviceArray.zeros((n_seq, n_rows, nq, hd), np.float32),
                                  pos=la.DeviceArray.from_numpy(self.pos0)))
        # algorithmic bytes of one step: each attended K and V byte once, Q read, O written
        self.kv_bytes = int(self.keys.sum()) * nkv * hd * 2 * 2
        self.qo_bytes = n_seq * n_rows * nq * hd * 4 * 2
        self.bytes = self.kv_bytes + self.qo_bytes
        self.flops = int(self.keys.sum()) * n_rows * nq * hd * 4  # upper bound for verify rows
        self._i = 0

    def step(self):
        st = self.sets[self._i % len(self.sets)]
        self._i += 1
        self.la.gqa_f16_varlen(st["q"], st["g"], True, st["kt"], st["vt"], st["pos"], st["out"],
                               self.n_seq, self.n_rows, self.keys_hint, self.nq, self.nkv, self.hd,
                               self.window, self.cap)

    def output(self, copy=0):
        return self.sets[copy]["out"].numpy()


class FusedStepWorkload(DecodeWorkload):
    """A decode step through lfm_hip_gqa_f16_step: the raw new-token q/k/v go
    through QK-RMSNorm (w = 1 + 0.05 N, eps 1e-5) + RoPE (theta 1e6) inside
    the attention kernel, which also stores the new K/V rows (config 2 as
    BASELINE defines it, prologue included).  Each step rewrites the same
    rows, so the bytes per step stay those of DecodeWorkload."""

    def __init__(self, la, rng, *a, **kw):
        super().__init__(la, rng, *a, **kw)
        hd = self.hd
        shape = (self.n_seq, self.n_rows, self.nkv, hd)
        self.k_raw = la.DeviceArray.from_numpy(rng.standard_normal(shape, dtype=np.float32))
        self.v_raw = la.DeviceArray.from_numpy(rng.standard_normal(shape, dtype=np.float32))
        self.qw = la.DeviceArray.from_numpy((1 + 0.05 * rng.standard_normal(hd)).astype(np.float32))
        self.kw = la.DeviceArray.from_numpy((1 + 0.05 * rng.standard_normal(hd)).astype(np.float32))
        c, s = la.rope_lut_lfm2(int(self.pos0.max()) + self.n_rows, hd, 1e6)
        self.cos, self.sin = la.DeviceArray.from_numpy(c), la.DeviceArray.from_numpy(s)

    def step(self):
        st = self.sets[self._i % len(self.sets)]
        self._i += 1
        self.la.gqa_f16_step(st["q"], self.k_raw, self.v_raw, st["g"], True, st["kt"], st["vt"], st["pos"],
                             st["out"], self.n_seq, self.n_rows, self.keys_hint, self.nq, self.nkv, self.hd,
                             self.qw, self.kw, 1e-5, self.cos, self.sin, self.window, self.cap)


def bench_engine_step(la, rng, nq=16, nkv=8, hd=64, pos=1023, calls=500):
    """lfm_attn_ctx_forward end to end, as the engine calls it per attention
    layer (host q/k/v in, host output out, synchronous): one host-to-device
    copy, the fused attention launch (+ split merge), one device-to-host
    copy.  Config 1's shape (16q/8kv d64, position 1023).  Wall clock per
    call, median of 5 batches of `calls`."""
    ctx = la.EngineContext(1, nq, nkv, hd, pos + 1, 1e-5, rope_base=1e6)
    try:
        ctx.set_norms(0, (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32),
                      (1 + 0.05 * rng.standard_normal(hd)).astype(np.float32))
        kv = (pos, nkv * hd)
        ctx.kv_import(0, 0, f16(rng.standard_normal(kv) * 0.5), f16(rng.standard_normal(kv) * 0.5))
        q = rng.standard_normal((1, nq, hd), dtype=np.float32)
        k = rng.standard_normal((1, nkv, hd), dtype=np.float32)
        v = rng.standard_normal((1, nkv, hd), dtype=np.float32)
        for _ in range(50):
            ctx.forward(0, pos, q, k, v)
        per = []
        for _ in range(5):
            t = time.perf_counter()
            for _ in range(calls):
                ctx.forward(0, pos, q, k, v)
            per.append((time.perf_counter() - t) / calls)
    finally:
        ctx.close()
    us = float(np.median(per)) * 1e6
    return dict(us_per_call=round(us, 2), shape=f"{nq}q/{nkv}kv d{hd}, position {pos}, one layer",
                includes="host->device copy, fused QK-norm+RoPE+K/V store+attention, merge, device->host copy, sync")


class PrefillWorkload:
    """causal prefill, B sequences of N tokens, fp16 Q/K/V
    (0.5*N(0,1), RoPE assumed applied), fp32 softmax/accumulate, fp32 out.
    The entry point takes Q as float (the reference's rows): the fp16 Q values
    are passed widened, exactly."""

    def __init__(self, la, rng, n_seq=4, n_tok=4096, nq=32, nkv=8, hd=64):
        self.la, self.n_seq, self.n_tok, self.nq, self.nkv, self.hd = la, n_seq, n_tok, nq, nkv, hd
        self.q = la.DeviceArray.from_numpy(
            f16(rng.standard_normal((n_seq, n_tok, nq, hd), dtype=np.float32) * np.float32(0.5))
            .view(np.float16).astype(np.float32))
        self.k = la.DeviceArray.from_numpy(
            f16(rng.standard_normal((n_seq, n_tok, nkv, hd), dtype=np.float32) * np.float32(0.5)))
        self.v = la.DeviceArray.from_numpy(
            f16(rng.standard_normal((n_seq, n_tok, nkv, hd), dtype=np.float32) * np.float32(0.5)))
        self.out = la.DeviceArray.zeros((n_seq, n_tok, nq, hd), np.float32)
        # causal algorithmic FLOPs: 2 GEMMs x 2 flop x d per (row, key <= row) per head
        self.flops = 4 * hd * nq * n_seq * n_tok * (n_tok + 1) // 2

    def step(self):
        self.la.prefill_f16(self.q, self.k, self.v, self.out, self.n_seq, self.n_tok, 0,
                            self.n_tok * self.nkv * self.hd, self.nq, self.nkv, self.hd)


class Lfm3PrefillWorkload:
    """LFM3 attention-layer prefill (lfm_hip_lfm3_prefill_f16): B sequences
    of N tokens, 16q/4kv, head_dim 128, gate logits N(0,1); a full layer
    (window 0) or a sliding-window layer (every row attends its last `window`
    positions).  Q/K/V as for config 4 (0.5*N(0,1), fp16 values)."""

    def __init__(self, la, rng, n_seq=4, n_tok=4096, nq=16, nkv=4, hd=128, window=0):
        self.la, self.n_seq, self.n_tok, self.nq, self.nkv, self.hd = la, n_seq, n_tok, nq, nkv, hd
        self.window = window
        self.q = la.DeviceArray.from_numpy(
            f16(rng.standard_normal((n_seq, n_tok, nq, hd), dtype=np.float32) * np.float32(0.5))
            .view(np.float16).astype(np.float32))
        self.k = la.DeviceArray.from_numpy(
            f16(rng.standard_normal((n_seq, n_tok, nkv, hd), dtype=np.float32) * np.float32(0.5)))
        self.v = la.DeviceArray.from_numpy(
            f16(rng.standard_normal((n_seq, n_tok, nkv, hd), dtype=np.float32) * np.float32(0.5)))
        self.gate = la.DeviceArray.from_numpy(rng.standard_normal((n_seq, n_tok, nq)).astype(np.float32))
        self.out = la.DeviceArray.zeros((n_seq, n_tok, nq, hd), np.float32)
        p = np.arange(n_tok, dtype=np.int64)
        keys = np.minimum(p + 1, window) if window else p + 1
        # 2 GEMMs x 2 flop x d per (row, attended key) per head
        self.flops = int(4 * hd * nq * n_seq * keys.sum())

    def step(self):
        self.la.lfm3_prefill_f16(self.q, self.k, self.v, self.gate, True, self.out, self.n_seq, self.n_tok, 0, 0,
                                 self.n_tok * self.nkv * self.hd, self.window, self.nq, self.nkv, self.hd)


class KvShiftWorkload:
    """Attention-sink eviction at the engine trigger (src/lfm2_api.c:871-891)
    for the LFM2-1.2B attention layers: 6 layers x 8 KV heads x d64 caches of
    max_seq 32768, position 32760, 64 sinks, n_discard = max_seq / 2.  Each
    step moves the same rows (the caches are overwritten in place), so the
    bytes per step are constant: every moved K and V byte is read and written."""

    def __init__(self, la, rng, n_layers=6, nkv=8, hd=64, max_seq=32768, n_sink=64):
        self.la = la
        row = nkv * hd
        self.k = [la.DeviceArray.from_numpy(f16(rng.standard_normal((max_seq, row), dtype=np.float32)))
                  for _ in range(n_layers)]
        self.v = [la.DeviceArray.from_numpy(f16(rng.standard_normal((max_seq, row), dtype=np.float32)))
                  for _ in range(n_layers)]
        c, s = la.rope_lut_lfm2(max_seq, hd, 1e6)
        self.cos, self.sin = la.DeviceArray.from_numpy(c), la.DeviceArray.from_numpy(s)
        self.args = (n_layers, nkv, hd, max_seq)
        self.pos, self.n_sink, self.n_discard = max_seq - 8, n_sink, max_seq // 2
        n_keep = self.pos - n_sink - self.n_discard
        self.bytes = 4 * n_layers * n_keep * row * 2

    def step(self):
        n_layers, nkv, hd, max_seq = self.args
        self.la.kv_cache_shift_sinks(self.k, self.v, [nkv] * n_layers, hd, self.cos, self.sin,
                                     max_seq, self.pos, self.n_sink, self.n_discard)


class FusedQkvWorkload:
    """LFM2-1.2B fused Q/K/V projection of one decode token: Q4_K 2048 x 2048
    (Q) and 512 x 2048 (K), Q6_K 512 x 2048 (V, as Q4_K_M files store it), one
    pass over the same Q8_K activations; rotated weight copies as in
    QuantProjWorkload."""

    def __init__(self, la, rng, n_tokens=1, copies=80):
        self.la, self.n_tokens = la, n_tokens
        self.rows, self.types, n_cols = [2048, 512, 512], [12, 12, 14], 2048
        self.n_cols = n_cols
        blk = {12: 144, 14: 210}
        mats = []
        for r, t in zip(self.rows, self.types):
            w = rng.integers(0, 256, size=(r, 8 * blk[t]), dtype=np.uint8)
            if t == 12:
                w.reshape(-1, 144)[:, 0:4] = np.array([0x2400, 0x2000], np.uint16).view(np.uint8)
            else:
                w.reshape(-1, 210)[:, 208:210] = np.array([0x2000], np.uint16).view(np.uint8)
            mats.append(w)
        self.w = [[la.DeviceArray.from_numpy(w) for w in mats] for _ in range(copies)]
        xd = la.DeviceArray.from_numpy(rng.standard_normal((n_tokens, n_cols)).astype(np.float32))
        self.xq = la.DeviceArray.zeros((n_tokens, 8 * 292), np.uint8)
        la.quantize_q8_K(xd, self.xq, n_tokens, n_cols)
        self.outs = [la.DeviceArray.zeros((n_tokens, r), np.float32) for r in self.rows]
        self.i = 0
        self.bytes = sum(m.nbytes for m in mats) + n_tokens * 8 * 292 + n_tokens * sum(self.rows) * 4

    def step(self):
        self.la.gqa_qkv_fused(self.outs, self.w[self.i], self.types, self.rows, self.n_cols, self.xq,
                              self.n_tokens)
        self.i = (self.i + 1) % len(self.w)


# bytes per 256 weights and the offsets of fp16 scale fields within each block
Q_LAYOUT = {2: (144, 18, (0,)), 8: (272, 34, (0,)), 12: (144, 144, (0, 2)), 13: (176, 176, (0, 2)),
            14: (210, 210, (208,)), 23: (136, 136, (0,))}


def random_q_rows(rng, qtype, n_rows, n_cols):
    """Random weight rows of a GGML type with small finite fp16 scales."""
    per256, blk, scale_offs = Q_LAYOUT[qtype]
    w = rng.integers(0, 256, size=(n_rows, n_cols // 256 * per256), dtype=np.uint8)
    b = w.reshape(-1, blk)
    for o in scale_offs:
        b[:, o:o + 2] = np.array([0x2000], np.uint16).view(np.uint8)
    return w


class QuantProjWorkload:
    """A quantized projection beside the attention path: LFM2-1.2B `wo`
    (2048 x 2048) applied to n_tokens Q8_K tokens, weights of GGML type qtype
    (Q4_K by default).  Each step reads a different copy of the weights, so
    the weights (not the 256 MB last-level cache) are streamed from HBM as at
    decode, where a step reads every layer's weights once."""

    def __init__(self, la, rng, n_rows=2048, n_cols=2048, n_tokens=1, copies=120, qtype=12):
        self.la, self.n_rows, self.n_cols, self.n_tokens = la, n_rows, n_cols, n_tokens
        self.qtype = qtype
        nb = n_cols // 256
        w = random_q_rows(rng, qtype, n_rows, n_cols)
        self.w = [la.DeviceArray.from_numpy(w) for _ in range(copies)]
        x = rng.standard_normal((n_tokens, n_cols)).astype(np.float32)
        xd = la.DeviceArray.from_numpy(x)
        self.xq = la.DeviceArray.zeros((n_tokens, nb * 292), np.uint8)
        la.quantize_q8_K(xd, self.xq, n_tokens, n_cols)
        self.out = la.DeviceArray.zeros((n_tokens, n_rows), np.float32)
        self.i = 0
        self.bytes = w.nbytes + n_tokens * nb * 292 + n_tokens * n_rows * 4

    def step(self):
        self.la.matmul_prequant(self.out, self.w[self.i], self.qtype, self.n_rows, self.n_cols, self.xq,
                                self.n_tokens)
        self.i = (self.i + 1) % len(self.w)


def bench_prompt_cache(la, rng, n_tokens=4096, reps=5):
    """.lfmcache v1 save and prefix load of an LFM2-1.2B session (16 layers:
    ShortConv states of 10, fp16 K/V of the 6 attention layers, 32q/8kv d64)
    at n_tokens positions, through the engine context; and the device FNV-1a
    64 over a payload of that size.  Times are wall clock around the host
    calls (file in the temp directory, fsync included)."""
    import tempfile

    kinds = [0] * 16
    for l in (2, 5, 8, 10, 12, 14):
        kinds[l] = 1
    ctx = la.EngineContext(6, 32, 8, 64, n_tokens)
    for l in range(6):
        ctx.kv_import(l, 0, rng.integers(0, 1 << 16, (n_tokens, 512), dtype=np.uint16),
                      rng.integers(0, 1 << 16, (n_tokens, 512), dtype=np.uint16))
    ctx_layer, i = [], 0
    for k in kinds:
        ctx_layer.append(i if k else -1)
        i += 1 if k else 0
    model = la.CacheModel(0x4C464D32315A4232, ctx_layer, 2048, 32, 3)  # the engine's fingerprint
    conv = [rng.standard_normal(2 * 2048).astype(np.float32) if k == 0 else None for k in kinds]
    tok = rng.integers(0, 65536, n_tokens, dtype=np.uint32)
    fd, path = tempfile.mkstemp(suffix=".lfmcache")
    os.close(fd)
    try:
        ctx.cache_save(path, model, tok, conv)
        size = os.path.getsize(path)
        dst = [None if c is None else np.zeros_like(c) for c in conv]
        saves, loads = [], []
        for _ in range(reps):
            t = time.perf_counter()
            ctx.cache_save(path, model, tok, conv)
            saves.append(time.perf_counter() - t)
            t = time.perf_counter()
            matched, _ = ctx.cache_load_prefix(path, model, tok, dst)
            loads.append(time.perf_counter() - t)
            assert matched == n_tokens
    finally:
        os.unlink(path)
        ctx.close()
    payload = size - 72
    buf = la.DeviceArray.from_numpy(rng.integers(0, 256, payload, dtype=np.uint8))
    la.fnv1a64(buf, payload)
    t = time.perf_counter()
    for _ in range(20):
        la.fnv1a64(buf, payload)
    h_s = (time.perf_counter() - t) / 20
    del buf
    ts, tl = float(np.median(saves)), float(np.median(loads))
    return dict(file_bytes=size, save_ms=round(ts * 1e3, 2), load_ms=round(tl * 1e3, 2),
                save_GBps=round(size / ts / 1e9, 2), load_GBps=round(size / tl / 1e9, 2),
                fnv1a64_device_ms=round(h_s * 1e3, 3), fnv1a64_device_GBps=round(payload / h_s / 1e9, 1))


SETTLE_S = 0.25  # clock settle before every timed row (time-based)


def settle(hip, wl, seconds=SETTLE_S):
    """Run the workload back to back for `seconds` of wall clock before its
    warm-up and timed steps: on MI355X the shader clock takes tens of
    milliseconds of sustained load to settle (the first ~60 config-4 prefill
    launches, ~20 ms, ran up to 20 % slower than later ones; the first 50
    headline steps after 10 warm-ups 7 % slower than after 300), so a fixed
    handful of warm-up steps starts the timed loop on an unsettled clock.
    Returns the launches it took."""
    n, t0 = 0, time.perf_counter()
    while True:
        for _ in range(8):
            wl.step()
        n += 8
        hip.sync()
        if time.perf_counter() - t0 >= seconds:
            return n


def time_steps(hip, wl, steps, warmup):
    """Settle, then `warmup` untimed steps, then the mean of exactly `steps`
    steps between two events on the launch stream."""
    settle(hip, wl)
    for _ in range(warmup):
        wl.step()
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0)
    for _ in range(steps):
        wl.step()
    hip.record(e1)
    hip.sync()
    return hip.elapsed_ms(e0, e1) / steps


# Launches of one step, by plan: split keys need the merge kernel after the
# attention kernel except in the in-workgroup form ("wg").
STEP_KERNELS = {"balanced": "k_splitkv_bal + k_merge_bal",
                "balanced-dma": "k_splitkv_bal (LDS-streamed segments) + k_merge_bal", "grid": "k_splitkv + k_merge (one launch when the "
                "keys are not split)", "wg": "k_splitkv_wg (merge inside the workgroup)", "generic": "k_generic"}


class _Probe:
    """One launch of a peak probe as a bench step."""

    def __init__(self, fn):
        self.step = fn


def box_peaks(hip, la, steps=10):
    """This device's achievable denominators: a 2 GiB streaming read (well
    past the 256 MB MALL) and a dense fp16 MFMA loop, both hand-written
    probes of the library (peak_probe.hip)."""
    from laii_amd._lib import check

    lib = la.load()
    n_bytes = 2 << 30
    src = la.DeviceArray.zeros(n_bytes // 4, np.uint32)
    # 2048 x 256 threads: one residency round (32 waves per CU); 8192
    # workgroups (four rounds) read 7 % slower on MI355X (6.69 vs 7.20 TB/s
    # over 1 GiB), 1024 slower still
    n_wg = 2048
    sink = la.DeviceArray.zeros(n_wg, np.uint32)
    rd = _Probe(lambda: check(lib.lfm_hip_probe_read(src.ptr, n_bytes, sink.ptr, n_wg, None),
                                 "lfm_hip_probe_read"))
    read_ms = min(time_steps(hip, rd, steps, 2) for _ in range(2))
    del src
    wgs, iters = 4096, 2048
    out = la.DeviceArray.zeros(wgs * 256, np.float32)
    mf = _Probe(lambda: check(lib.lfm_hip_probe_mfma(out.ptr, wgs, iters, None), "lfm_hip_probe_mfma"))
    mfma_ms = min(time_steps(hip, mf, steps, 2) for _ in range(2))
    flops = wgs * 4 * iters * 8 * 16384
    return dict(read_GBps=round(n_bytes / (read_ms * 1e-3) / 1e9, 1),
                mfma_f16_TFLOPs=round(flops / (mfma_ms * 1e-3) / 1e12, 1),
                read="2 GiB streaming read, 2048 x 256 threads, 16-B nontemporal loads",
                mfma="4096 x 4 waves, 8 independent 16x16x32 f16 MFMA chains per wave")


CPU_WARM, CPU_REPS = 3, 10  # the benchmark method: median of >= 10 timed passes after 3 warm-ups


def _cpu_legs(ref, kind, q, k_list, v_list, pos0, nq, nkv, hd, n_threads, algo, unit, **kw):
    """Both legs of one configuration on the reference's own CPU kernels
    (oracle/_ref): the engine's dispatch per sequence (per row) on a pool of
    n_threads ("reference_faithful") and every (sequence, row, item) of the
    sample claimed by n_threads threads ("fair_batched").  algo: the sample's
    algorithmic bytes or FLOPs; unit "GB/s" or "TFLOP/s".  Medians of
    CPU_REPS passes after CPU_WARM warm-ups."""
    legs, out, used = {}, None, 0
    for name, fair in (("reference_faithful", False), ("fair_batched", True)):
        times, used, o = ref.time_attn(kind, fair, q, k_list, v_list, pos0, nq, nkv, hd, n_threads=n_threads,
                                       warm=CPU_WARM, reps=CPU_REPS, **kw)
        med = float(np.median(times))
        rate = algo / med / (1e9 if unit == "GB/s" else 1e12)
        legs[name] = {"value": round(rate, 4), "unit": unit, "ms_per_pass": round(med * 1e3, 3),
                      "spread_ms": [round(float(times.min()) * 1e3, 3), round(float(times.max()) * 1e3, 3)]}
        if out is None:
            out = o
    legs["cores"] = int(used)
    return legs, out


def _kv_sample(rng, n_slots, nkv, hd):
    return [f16(rng.standard_normal((n, nkv, hd), dtype=np.float32) * np.float32(0.5)) for n in n_slots]


def cpu_baseline(wl, n_threads):
    """The headline's CPU baseline: the reference's AVX2 decode worker
    (oracle/_ref) on 8 of the 64 sequences, both legs; the C restatement
    (kind "port") where the reference build is absent."""
    from oracle.bindings import Oracle, Reference

    n = len(wl.host_k)
    q = wl.host_q[:n, 0].reshape(n, -1)
    pos = wl.pos0[:n]
    sample_bytes = int(wl.keys[:n].sum()) * wl.nkv * wl.hd * 4 + n * wl.nq * wl.hd * 8
    sample = f"{n} of {wl.n_seq} sequences x ctx {int(wl.keys[0])}, 32q/8kv d64"
    if Reference.available():
        legs, out = _cpu_legs(Reference(), "lfm2_decode", q, wl.host_k, wl.host_v, pos, wl.nq, wl.nkv, wl.hd,
                              n_threads, sample_bytes, "GB/s")
        rf, fb = legs["reference_faithful"], legs["fair_batched"]
        res = dict(value=rf["value"], unit="GB/s", cores=legs["cores"], kind="reference",
                   sample=f"{sample}, dispatched per sequence as the engine does (ceil(32/4) head-group items on "
                          f"one pool), median of {CPU_REPS} passes after {CPU_WARM} warm-ups, "
                          f"{rf['ms_per_pass']} ms per pass",
                   fair_batched=dict(value=fb["value"], unit="GB/s", cores=legs["cores"], kind="reference",
                                     sample=f"same sample, every (sequence, head group) item on all threads, "
                                            f"{fb['ms_per_pass']} ms per pass"))
    else:
        orc = Oracle()
        t0 = time.perf_counter()
        out = orc.decode_batch_mt(q, wl.host_k, wl.host_v, pos, wl.nq, wl.nkv, wl.hd, n_threads)
        dt = time.perf_counter() - t0
        res = dict(value=round(sample_bytes / dt / 1e9, 3), unit="GB/s", cores=n_threads, kind="port",
                   sample=f"{sample}, one pass of the C restatement")
    res["method"] = f"median of {CPU_REPS} timed passes after {CPU_WARM} warm-up passes"
    res["host"] = host_cpu()
    return res, out.reshape(n, wl.nq, wl.hd)


def cpu_config_rows(rng, n_threads, ragged_ctx):
    """Both CPU legs for every other BASELINE configuration, on bounded
    samples of the GPU rows' shapes and input distribution (fp16 K/V
    0.5*N(0,1), N(0,1) queries, sigmoid of N(0,1) gate logits); {} when the
    reference build is absent."""
    from oracle.bindings import Reference

    if not Reference.available():
        return {}
    ref = Reference()
    rows = {}

    def decode_row(name, kind, n_seq_total, ctx, nq, nkv, hd, note, window=0, cap=0, gate=False, n_rows=1):
        ctx = np.asarray(ctx, np.int64)
        n = len(ctx)
        if n_rows > 1:   # verify rows: row r of a sequence at ctx + r
            pos0, slots = ctx, ctx + n_rows
            keys = int(sum(int(c) + n_rows for c in ctx))                   # K/V read once per sequence
            flops = int(sum(4 * hd * nq * (int(c) + r + 1) for c in ctx for r in range(n_rows)))
        else:
            pos0 = ctx - 1
            slots = np.full(n, cap) if window else ctx
            keys = int(sum(min(int(c), window) if window else int(c) for c in ctx))
            flops = 4 * hd * nq * keys
        kl, vl = _kv_sample(rng, [int(x) for x in slots], nkv, hd), _kv_sample(rng, [int(x) for x in slots], nkv, hd)
        q = rng.standard_normal((n, n_rows, nq, hd), dtype=np.float32)
        g = (1.0 / (1.0 + np.exp(-rng.standard_normal((n, nq))))).astype(np.float32) if gate else None
        algo = keys * nkv * hd * 4 + n * n_rows * nq * hd * 8
        legs, _ = _cpu_legs(ref, kind, q, kl, vl, pos0.astype(np.uint32), nq, nkv, hd, n_threads, algo, "GB/s",
                            n_rows=n_rows, gate=g, window=window, cap=cap)
        legs.update(kind="reference", sample=f"{n} of {n_seq_total} sequences, {note}", algorithmic_bytes=algo,
                    flops=flops)
        rows[name] = legs

    decode_row("cfg1_decode_b1_16q8kv_ctx1024", "lfm2_decode", 1, [1024], 16, 8, 64,
               "16q/8kv d64 at position 1023, lfm2_online_gqa_f16_worker_simd over ceil(16/4) items")
    decode_row("cfg2_varlen_b64_ctxU512_8192", "lfm2_decode", 64, list(ragged_ctx[:8]), 32, 8, 64,
               "the GPU row's first 8 contexts, 32q/8kv d64, per-sequence M=1 dispatch")
    decode_row("cfg3_verify_b16_rows8_ctx4096", "lfm2_rows", 16, [4096] * 2, 32, 8, 64,
               "8 causal rows over 4096 + 8 keys, lfm2_gqa_heads_worker_task per row (the verify path)", n_rows=8)
    decode_row("cfg5_lfm3_swa_b32_cap256_pos1000", "lfm3_decode", 32, [1001] * 32, 16, 4, 128,
               "window 256 in a 256-slot ring at position 1000, gate, lfm3_online_gqa_f16_dispatch (B = 1)",
               window=256, cap=256, gate=True)
    decode_row("cfg5_lfm3_full_b32_ctx32768", "lfm3_decode", 32, [32768] * 2, 16, 4, 128,
               "full layer at position 32767, gate, lfm3_online_gqa_f16_dispatch (B = 1)", gate=True)
    # config 4: 64 prefill rows of one sequence at positions 63 .. 4095 (one
    # pseudo-sequence per row over the same cache), per-row heads dispatch
    n_tok, nq, nkv = 4096, 32, 8
    k16, v16 = _kv_sample(rng, [n_tok], nkv, 64)[0], _kv_sample(rng, [n_tok], nkv, 64)[0]
    pos = np.arange(63, n_tok, 64, dtype=np.uint32)
    q = (rng.standard_normal((pos.size, nq * 64)) * 0.5).astype(np.float16).astype(np.float32)
    flops = float(sum(4 * 64 * nq * (int(p) + 1) for p in pos))
    legs, _ = _cpu_legs(ref, "lfm2_rows", q, [k16] * pos.size, [v16] * pos.size, pos, nq, nkv, 64, n_threads,
                        flops, "TFLOP/s")
    legs.update(kind="reference", flops=flops,
                sample=f"{pos.size} rows at positions 63..4095 of config 4, lfm2_gqa_heads_worker_task per row "
                       f"(one row per dispatch, as lfm2_forward_gqa_batch runs them)")
    rows["prefill_cfg4_rows"] = legs
    return rows


def host_cpu():
    """CPU model, logical CPUs and physical cores of the timing host."""
    model, cores = None, set()
    try:
        phys = core = None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model is None:
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None:
                cores.add((phys, core))
                phys = core = None
    except OSError:
        pass
    return dict(model=model, logical_cpus=os.cpu_count(), physical_cores=len(cores) or None,
                affinity_cpus=len(os.sched_getaffinity(0)))


def cpu_prompt_cache(rng, n_tokens=4096, reps=3):
    """The reference's .lfmcache writer and prefix loader (oracle/_ref; the C
    restatement when absent) on host caches of the bench_prompt_cache layout."""
    import tempfile

    from oracle.bindings import CacheModel, Oracle, Reference

    kinds = [0] * 16
    for l in (2, 5, 8, 10, 12, 14):
        kinds[l] = 1
    m = CacheModel(kinds, [8 if k else 0 for k in kinds], 64, 2048, 32, 3)
    lib, kind = (Reference(), "reference") if Reference.available() else (Oracle(), "port")
    conv = [rng.standard_normal(2 * 2048).astype(np.float32) if k == 0 else None for k in kinds]
    k = [rng.integers(0, 1 << 16, n_tokens * 512, dtype=np.uint16) if x else None for x in kinds]
    v = [rng.integers(0, 1 << 16, n_tokens * 512, dtype=np.uint16) if x else None for x in kinds]
    tok = rng.integers(0, 65536, n_tokens, dtype=np.uint32)
    fd, path = tempfile.mkstemp(suffix=".lfmcache")
    os.close(fd)
    saves, loads = [], []
    try:
        for _ in range(reps):
            t = time.perf_counter()
            assert lib.prompt_cache_save(path, m, tok, conv, k, v)
            saves.append(time.perf_counter() - t)
            t = time.perf_counter()
            assert lib.prompt_cache_load(path, m, tok, n_tokens, conv, k, v)[0] == n_tokens
            loads.append(time.perf_counter() - t)
    finally:
        os.unlink(path)
    return dict(save_ms=round(float(np.median(saves)) * 1e3, 2), load_ms=round(float(np.median(loads)) * 1e3, 2),
                cores=1, kind=kind, sample=f"LFM2-1.2B session at {n_tokens} tokens, median of {reps}")


def cpu_rows(rng, n_threads):
    """The reference's CPU path for the rows beside attention, on bounded
    samples (oracle/_ref; skipped when the reference build is absent): LFM2
    attention-sink eviction, the Q4_K `wo` projection."""
    from oracle.bindings import Reference

    if not Reference.available():
        return {}
    ref = Reference()
    rows = {}
    # sink eviction: 6 layers x 8 KV heads x d64, max_seq 16384, position 16376, 64 sinks
    max_seq, n_layers, pos0, n_sink = 16384, 6, 16376, 64
    lut = ref.rope_lut_lfm2(max_seq, 64, 1e6)
    kc = [(rng.standard_normal((max_seq, 512)) * 0.5).astype(np.float16).view(np.uint16) for _ in range(n_layers)]
    vc = [(rng.standard_normal((max_seq, 512)) * 0.5).astype(np.float16).view(np.uint16) for _ in range(n_layers)]
    t = time.perf_counter()
    ref.kv_shift_sinks_lfm2(kc, vc, [8] * n_layers, 64, lut, pos0, n_sink, max_seq // 2)
    dt = time.perf_counter() - t
    moved = 4 * n_layers * (pos0 - n_sink - max_seq // 2) * 512 * 2
    rows["kv_shift_sinks_lfm2"] = dict(GBps=round(moved / dt / 1e9, 2), cores=1, kind="reference",
                                       sample=f"6 layers, max_seq {max_seq} at position {pos0}, {dt * 1e3:.1f} ms")
    # `wo`: Q4_K 2048 x 2048, one token, the engine's decode projection without a pool
    w = rng.integers(0, 256, size=(2048, 8 * 144), dtype=np.uint8)
    w.reshape(-1, 144)[:, 0:4] = np.array([0x2400, 0x2000], np.uint16).view(np.uint8)
    xq = ref.quantize_q8_K(rng.standard_normal((1, 2048)).astype(np.float32))
    ref.matmul_q4_K_prequant(w, xq, 2048)
    t = time.perf_counter()
    for _ in range(20):
        ref.matmul_q4_K_prequant(w, xq, 2048)
    dt = (time.perf_counter() - t) / 20
    rows["wo_q4K_q8K_tokens1"] = dict(us=round(dt * 1e6, 1), GBps=round(w.nbytes / dt / 1e9, 2), cores=1,
                                      kind="reference", sample="2048 x 2048 Q4_K, lfm2_matmul_1x4_prequant_mt")
    return rows


def decode_cases(rng):
    """The secondary decode / verify / LFM3 workloads (name, DecodeWorkload
    arguments)."""
    return [
        ("cfg2_varlen_b64_ctxU512_8192", dict(n_seq=64, n_rows=1, nq=32, nkv=8, hd=64,
                                              ctx=rng.integers(512, 8193, size=64))),
        ("cfg3_verify_b16_rows8_ctx4096", dict(n_seq=16, n_rows=8, nq=32, nkv=8, hd=64,
                                               ctx=[4096] * 16, copies=4)),
        ("cfg5_lfm3_swa_b32_cap256_pos1000", dict(n_seq=32, n_rows=1, nq=16, nkv=4, hd=128,
                                                  ctx=[1001] * 32, window=256, cap=256,
                                                  gate=True, copies=36)),
        ("cfg5_lfm3_full_b32_ctx32768", dict(n_seq=32, n_rows=1, nq=16, nkv=4, hd=128,
                                             ctx=[32768] * 32, gate=True)),
        # 2 MB per call: 160 rotated copies (320 MB) keep it out of the 256 MB
        # MALL; the row is latency-bound, so us_per_step is its figure
        ("cfg1_decode_b1_16q8kv_ctx1024", dict(n_seq=1, n_rows=1, nq=16, nkv=8, hd=64,
                                               ctx=[1024], copies=160)),
    ]


def prefill_counts(steps, warmup):
    """Timed launches and warm-up launches of a prefill row (each ~0.3 ms,
    after the time-based settle)."""
    return max(10, steps // 2), warmup


def run_prefill(hip, la, rng, steps, warmup):
    pf = PrefillWorkload(la, rng)
    n, w = prefill_counts(steps, warmup)
    pms = time_steps(hip, pf, n, w)
    prefill = dict(workload="cfg4_prefill_b4_n4096_32q8kv_d64", TFLOPs=round(pf.flops / (pms * 1e-3) / 1e12, 1),
                   ms_per_step=round(pms, 4), flops=pf.flops,
                   pct_fp16_mfma_peak=round(100 * pf.flops / (pms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFS, 1),
                   kernel="k_prefill<64> (one launch per step)", launches=n, warmup_launches=w,
                   settle_s=SETTLE_S)
    log(f"prefill: {pms:.3f} ms/step, {prefill['TFLOPs']} TFLOP/s")
    return prefill


def run_prefill_lfm3(hip, la, rng, steps, warmup, window):
    pf = Lfm3PrefillWorkload(la, rng, window=window)
    n, w = prefill_counts(steps, warmup)
    pms = time_steps(hip, pf, n, w)
    kind = f"swa{window}" if window else "full"
    row = dict(workload=f"lfm3_{kind}_prefill_b4_n4096_16q4kv_d128_gate", TFLOPs=round(pf.flops / (pms * 1e-3) / 1e12, 1),
               ms_per_step=round(pms, 4), flops=pf.flops,
               pct_fp16_mfma_peak=round(100 * pf.flops / (pms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFS, 1),
               kernel="k_prefill_ext<128> (one launch per step)", launches=n, warmup_launches=w)
    log(f"lfm3 {kind} prefill: {pms:.3f} ms/step, {row['TFLOPs']} TFLOP/s")
    del pf
    return row


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # warm-up long enough for the clocks to settle: on MI355X the first 50
    # timed headline steps ran 183 us after 10 warm-up steps and 171-172 us
    # after 100-300 (steady state 170.5 us)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--quick", action="store_true", help="headline only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the config-4 prefill workload (for kernel profiling)")
    ap.add_argument("--prefill128-only", action="store_true",
                    help="only the LFM3 head_dim-128 prefill workloads (for kernel profiling)")
    ap.add_argument("--window", type=int, default=None,
                    help="with --prefill128-only: only the row of this window (0 = the full layer)")
    ap.add_argument("--only", default=None,
                    help="only the named decode / verify / LFM3 workload of the secondary rows "
                         "(for kernel profiling), e.g. cfg3_verify_b16_rows8_ctx4096")
    ap.add_argument("--engine-only", action="store_true",
                    help="only the engine step, lfm_attn_ctx_forward (for kernel tracing)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share only; --gpus {args.gpus} is not supported: "
              "this build runs on one GPU (sequences or KV heads would shard across GPUs "
              "with no exchange, each GPU running this same single-GPU path)", file=sys.stderr)
        sys.exit(2)

    import laii_amd as la

    la.require_gpu()
    hip = Hip()
    rng = np.random.default_rng(20261201)
    t_setup = time.perf_counter()
    if args.only:
        kw = dict(decode_cases(rng))[args.only]
        wl = DecodeWorkload(la, rng, args.only, **kw)
        sms = time_steps(hip, wl, args.steps, args.warmup)
        print(json.dumps({"metric": f"{args.only} GB/s", "value": round(wl.bytes / (sms * 1e-3) / 1e9, 1),
                          "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "higher_is_better": True,
                          "us_per_step": round(sms * 1e3, 2), "plan": la.last_plan(), "bytes": wl.bytes}),
              flush=True)
        return
    if args.engine_only:
        es = bench_engine_step(la, rng, calls=max(10, args.steps))
        print(json.dumps({"metric": "engine attention step, host in/out", "value": es["us_per_call"],
                          "unit": "us", "n_gpus": 1, "higher_is_better": False, "engine_step": es}), flush=True)
        return
    if args.prefill128_only:
        windows = (0, 256) if args.window is None else (args.window,)
        rows = [run_prefill_lfm3(hip, la, rng, args.steps, args.warmup, w) for w in windows]
        print(json.dumps({"metric": "LFM3 prefill attn TFLOP/s, B4 x 4096, 16q/4kv d128", "value": rows[0]["TFLOPs"],
                          "unit": "TFLOP/s", "n_gpus": 1, "steps": prefill_counts(args.steps, args.warmup)[0],
                          "higher_is_better": True, "prefill_lfm3": rows}), flush=True)
        return
    if args.prefill_only:
        prefill = run_prefill(hip, la, rng, args.steps, args.warmup)
        print(json.dumps({"metric": "prefill attn TFLOP/s, config 4", "value": prefill["TFLOPs"],
                          "unit": "TFLOP/s", "n_gpus": 1, "steps": prefill_counts(args.steps, args.warmup)[0],
                          "higher_is_better": True, "prefill": prefill}), flush=True)
        return

    cases = decode_cases(rng)
    ragged_ctx = dict(cases)["cfg2_varlen_b64_ctxU512_8192"]["ctx"]
    head = DecodeWorkload(la, rng, "decode_b64_ctx8192", 64, 1, 32, 8, 64, [8192] * 64,
                          keep_host=8)
    log(f"headline inputs ready ({time.perf_counter() - t_setup:.1f} s)")
    ms = time_steps(hip, head, args.steps, args.warmup)
    head_plan = la.last_plan()
    log(f"headline: {ms * 1e3:.1f} us/step ({head_plan})")
    value = head.bytes / (ms * 1e-3) / 1e9
    achieved = value  # the attention step over the timed region (see roofline.timing)
    gpu_out = head.output()

    secondary = {}
    if not args.quick:
        for name, kw in cases:
            wl = DecodeWorkload(la, rng, name, **kw)
            sms = time_steps(hip, wl, args.steps, args.warmup)
            plan = la.last_plan()
            log(f"{name}: {sms * 1e3:.1f} us/step ({plan})")
            secondary[name] = dict(GBps=round(wl.bytes / (sms * 1e-3) / 1e9, 1),
                                   us_per_step=round(sms * 1e3, 2), bytes=wl.bytes,
                                   pct_hbm_peak=round(100 * wl.bytes / (sms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
                                   plan=plan, step=STEP_KERNELS.get(plan, plan))
            del wl

    if not args.quick:
        # config 2 as BASELINE defines it: the QK-norm + RoPE prologue of the
        # new token inside the attention kernel, which also stores its K/V
        for name, ctx in (("cfg2_fused_step_b64_ctx8192", [8192] * 64),
                          ("cfg2_fused_step_b64_ctxU512_8192", rng.integers(512, 8193, size=64))):
            wl = FusedStepWorkload(la, rng, name, 64, 1, 32, 8, 64, ctx)
            sms = time_steps(hip, wl, args.steps, args.warmup)
            plan = la.last_plan()
            log(f"{name}: {sms * 1e3:.1f} us/step ({plan})")
            secondary[name] = dict(GBps=round(wl.bytes / (sms * 1e-3) / 1e9, 1),
                                   us_per_step=round(sms * 1e3, 2), bytes=wl.bytes,
                                   pct_hbm_peak=round(100 * wl.bytes / (sms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
                                   plan=plan, step=STEP_KERNELS.get(plan, plan))
            del wl
        es = bench_engine_step(la, rng)
        secondary["engine_step_cfg1_host_in_out"] = es
        log(f"engine step (host in/out): {es['us_per_call']} us per call")

    prefill = run_prefill(hip, la, rng, args.steps, args.warmup)
    for w in (0, 256):
        row = run_prefill_lfm3(hip, la, rng, args.steps, args.warmup, w)
        secondary[row["workload"]] = row

    if not args.quick:
        ks = KvShiftWorkload(la, rng)
        kms = time_steps(hip, ks, max(5, args.steps // 5), 2)
        secondary["kv_shift_sinks_lfm2_1p2b_6layers_ctx32768"] = dict(
            GBps=round(ks.bytes / (kms * 1e-3) / 1e9, 1), us_per_step=round(kms * 1e3, 2), bytes=ks.bytes,
            pct_hbm_peak=round(100 * ks.bytes / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1))
        log(f"kv shift: {kms * 1e3:.1f} us/step")
        del ks
        for n_tok in (1, 64):
            qp = QuantProjWorkload(la, rng, n_tokens=n_tok)
            qms = time_steps(hip, qp, max(20, args.steps), 5)
            secondary[f"wo_q4K_q8K_lfm2_1p2b_2048x2048_tokens{n_tok}"] = dict(
                GBps=round(qp.bytes / (qms * 1e-3) / 1e9, 1), us_per_step=round(qms * 1e3, 2),
                bytes=qp.bytes, pct_hbm_peak=round(100 * qp.bytes / (qms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1))
            log(f"wo q4_K tokens {n_tok}: {qms * 1e3:.2f} us/step")
            del qp
        names = {2: "q4_0", 8: "q8_0", 13: "q5K", 14: "q6K", 23: "iq4xs"}
        types = {}
        for qtype in (2, 8, 13, 14, 23):
            qp = QuantProjWorkload(la, rng, n_tokens=1, qtype=qtype)
            qms = time_steps(hip, qp, max(20, args.steps), 5)
            types[names[qtype]] = dict(us_per_step=round(qms * 1e3, 2), bytes=qp.bytes,
                                       GBps=round(qp.bytes / (qms * 1e-3) / 1e9, 1))
            del qp
        secondary["wo_other_types_lfm2_1p2b_2048x2048_tokens1"] = types
        log("wo other types tokens 1: " + ", ".join(f"{k} {v['us_per_step']} us" for k, v in types.items()))
        fq = FusedQkvWorkload(la, rng)
        fms = time_steps(hip, fq, max(20, args.steps), 5)
        secondary["qkv_fused_q4K_q6K_lfm2_1p2b_tokens1"] = dict(
            GBps=round(fq.bytes / (fms * 1e-3) / 1e9, 1), us_per_step=round(fms * 1e3, 2), bytes=fq.bytes,
            pct_hbm_peak=round(100 * fq.bytes / (fms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1))
        log(f"qkv fused tokens 1: {fms * 1e3:.2f} us/step")
        del fq
        pc = bench_prompt_cache(la, rng)
        secondary["lfmcache_save_load_lfm2_1p2b_n4096"] = pc
        log(f"prompt cache: save {pc['save_ms']} ms, load {pc['load_ms']} ms, "
            f"device FNV-1a {pc['fnv1a64_device_GBps']} GB/s")

    peaks = None
    if not args.quick:
        peaks = box_peaks(hip, la)
        peaks["headline_frac_of_read"] = round(achieved / peaks["read_GBps"], 3)
        if prefill:
            peaks["prefill_frac_of_mfma"] = round(prefill["TFLOPs"] / peaks["mfma_f16_TFLOPs"], 3)
        log(f"box peaks: read {peaks['read_GBps']} GB/s, fp16 MFMA {peaks['mfma_f16_TFLOPs']} TFLOP/s")

    cpu = None
    parity = None
    if not args.no_cpu:
        n_thr = max(1, min(16, os.cpu_count() or 1) - 1)  # reference policy: N_phys - 1
        log(f"cpu baseline with {n_thr} threads")
        cpu, cpu_out = cpu_baseline(head, n_thr)
        if not args.quick:
            cpu["rows"] = cpu_config_rows(rng, n_thr, ragged_ctx)
            cpu["rows"]["lfmcache_save_load_lfm2_1p2b_n4096"] = cpu_prompt_cache(rng)
            cpu["rows"].update(cpu_rows(rng, n_thr))
            # GPU rate over the CPU legs' rates, per configuration
            for name, row in cpu["rows"].items():
                g = secondary.get(name, {}).get("GBps")
                if name == "prefill_cfg4_rows" and prefill:
                    g = prefill["TFLOPs"]
                if g and "reference_faithful" in row:
                    row["gpu_over_cpu"] = {k: round(g / row[k]["value"], 1)
                                           for k in ("reference_faithful", "fair_batched")}
        g = gpu_out[:cpu_out.shape[0], 0]
        parity = dict(max_abs=float(np.abs(g - cpu_out).max()),
                      rel_l2=float(np.linalg.norm(g - cpu_out) / np.linalg.norm(cpu_out)),
                      vs=cpu["kind"], sequences=int(cpu_out.shape[0]))

    line = {
        "metric": "decode attn KV GB/s (% HBM peak) + prefill attn TFLOP/s, LFM2-1.2B GQA shape",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV / f32 softmax+accumulate",
        "data": "synthetic, seeded N(0,1) Q and 0.5*N(0,1) fp16 K/V",
        "config": {"workload": "decode_b64_ctx8192", "n_seq": 64, "n_head_q": 32, "n_head_kv": 8,
                   "head_dim": 64, "ctx": 8192, "kv_bytes": head.kv_bytes,
                   "algorithmic_bytes": head.bytes},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": HEADLINE_TRAFFIC_BYTES,
                     "traffic_source": "constant from the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of "
                                       "profiles/k_splitkv_decode_b64_ctx8192_pmc.md, not measured in this run",
                     "kernel": "k_splitkv_bal<64,1,8,false> + k_merge_bal<64> (one attention step)",
                     "kernel_us": round(ms * 1e3, 2),
                     "timing": "HIP events on the launch stream around the timed region of `steps` steps, after "
                               f"a {SETTLE_S} s clock settle and `warmup` steps; each step is the split-KV kernel "
                               "and its merge, so kernel_us is the mean step (per-launch event brackets, which add "
                               "~5-7 us per launch, are not used)"},
        "clock_settle_s": SETTLE_S,
        "prefill": prefill,
        "box_peaks": peaks,
        "cpu_baseline": cpu,
        "parity_vs_cpu": parity,
        "secondary": secondary,
        "setup_s": round(time.perf_counter() - t_setup, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
