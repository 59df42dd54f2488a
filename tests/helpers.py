"""Shared input builders and the parity bar for the tests."""
from __future__ import annotations

import numpy as np

# fp32 outputs within max-abs 2e-3 and relative L2 1e-3
# of the CPU reference on the same inputs.
MAX_ABS = 2e-3
REL_L2 = 1e-3


def plan_overrides(la, env):
    """la.tuning(...) for a case named in the LFM_ATTN_* variable form
    ({"LFM_ATTN_PLAN": "grid", "LFM_ATTN_CHUNK": "96"}); {} = automatic."""
    return la.tuning(env.get("LFM_ATTN_PLAN"), int(env.get("LFM_ATTN_WAVES", 0)),
                     int(env.get("LFM_ATTN_CHUNK", 0)), int(env.get("LFM_ATTN_MINTILES", 0)))


def f16(x: np.ndarray) -> np.ndarray:
    """IEEE binary16 bits of x, round-to-nearest-even (numpy's cast is RNE)."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def rand_kv(rng, n_slots, n_kv, hd, scale=0.5):
    """fp16 cache [n_slots][n_kv][hd] of scale * N(0,1)."""
    return f16(rng.standard_normal((n_slots, n_kv, hd), dtype=np.float32) * np.float32(scale))


def parity(got, want, max_abs=MAX_ABS, rel_l2=REL_L2, what=""):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    assert got.shape == want.shape
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = float(np.abs(got - want).max()) if got.size else 0.0
    den = float(np.linalg.norm(want))
    rel = float(np.linalg.norm(got - want) / den) if den > 0 else err
    print(f"{what}: max_abs={err:.3e} rel_l2={rel:.3e}")
    assert err <= max_abs and rel <= rel_l2, f"{what}: max_abs={err:.3e} rel_l2={rel:.3e}"
    return err, rel


def softmax_attention_f64(q, k, v, scale):
    """Textbook softmax(scale * q.k) v in float64 for one head.
    q: [hd]; k, v: [n_keys, hd] (already dequantised)."""
    s = (k.astype(np.float64) @ q.astype(np.float64)) * float(scale)
    s -= s.max()
    p = np.exp(s)
    return (p @ v.astype(np.float64)) / p.sum()


# ---- GGUF Q4_K / Q8_K blocks (packed, as the reference's block_q4_K_t /
# block_q8_K_t, tools/lfm2_cpuid_quants.c:76-127) -----------------------------
Q4K_BYTES, Q8K_BYTES = 144, 292


def q4k_pattern(n_rows, nb, d, dmin, a, b, c, e):
    """The reference tests' deterministic Q4_K weights: block i has d, dmin,
    scales[j] = (i*a + j*b) & 63, qs[j] = (i*c + j*e) & 255."""
    n = n_rows * nb
    i = np.arange(n, dtype=np.int64)[:, None]
    blk = np.zeros((n, Q4K_BYTES), np.uint8)
    blk[:, 0:2] = np.array([d], np.uint16).view(np.uint8)
    blk[:, 2:4] = np.array([dmin], np.uint16).view(np.uint8)
    blk[:, 4:16] = ((i * a + np.arange(12) * b) & 0x3F).astype(np.uint8)
    blk[:, 16:144] = ((i * c + np.arange(128) * e) & 0xFF).astype(np.uint8)
    return blk.reshape(n_rows, nb * Q4K_BYTES)


def q4k_random(rng, n_rows, n_cols):
    """Random Q4_K rows: every bit of scales and qs random; d, dmin in
    [2^-10, 2^-6] as fp16."""
    nb = n_cols // 256
    blk = rng.integers(0, 256, size=(n_rows * nb, Q4K_BYTES), dtype=np.uint8)
    d = rng.uniform(2.0 ** -10, 2.0 ** -6, size=n_rows * nb).astype(np.float16)
    dm = rng.uniform(2.0 ** -10, 2.0 ** -6, size=n_rows * nb).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blk[:, 2:4] = dm.view(np.uint8).reshape(-1, 2)
    return blk.reshape(n_rows, nb * Q4K_BYTES)


def _q4k_scale_min(q, j, planted_error=False):
    if j < 4:
        return q[:, j] & 63, q[:, j + 4] & 63
    hi_src = q[:, j] if planted_error else q[:, j - 4]
    sc = (q[:, j + 4] & 0x0F) | ((hi_src >> 6) << 4)
    m = (q[:, j + 4] >> 4) | ((q[:, j] >> 6) << 4)
    return sc, m


def q4k_dequant(w, n_cols, planted_error=False):
    """float64 [n_rows, n_cols]: weight = d*sc*q - dmin*m of its sub-block
    (sub-block j of a super-block: nibbles of qs[32*(j//2) .. +32], low for
    even j, high for odd j)."""
    n_rows = w.shape[0]
    nb = n_cols // 256
    blk = w.reshape(n_rows * nb, Q4K_BYTES)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dm = blk[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    sc_bytes = blk[:, 4:16].astype(np.int64)
    qs = blk[:, 16:144].astype(np.int64)
    out = np.zeros((n_rows * nb, 256))
    for j in range(8):
        sc, m = _q4k_scale_min(sc_bytes, j, planted_error)
        q = qs[:, 32 * (j // 2):32 * (j // 2) + 32]
        nib = (q & 0x0F) if j % 2 == 0 else (q >> 4)
        out[:, 32 * j:32 * j + 32] = (d * sc)[:, None] * nib - (dm * m)[:, None]
    return out.reshape(n_rows, n_cols)


def q8k_dequant(q, n_cols):
    """Q8_K rows -> (float64 values d*q8 [n_rows, n_cols], d [n_rows, nb])."""
    n_rows = q.shape[0]
    nb = n_cols // 256
    blk = q.reshape(n_rows * nb, Q8K_BYTES)
    d = blk[:, 0:4].copy().view(np.float32).astype(np.float64)[:, 0]
    qs = blk[:, 4:260].copy().view(np.int8).astype(np.float64)
    return (qs * d[:, None]).reshape(n_rows, n_cols), d.reshape(n_rows, nb)


Q6K_BYTES = 210


def q6k_random(rng, n_rows, n_cols):
    """Random Q6_K rows: ql, qh random; int8 scales in [-64, 63]; d in [2^-12, 2^-8]."""
    nb = n_cols // 256
    blk = rng.integers(0, 256, size=(n_rows * nb, Q6K_BYTES), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-64, 64, size=(n_rows * nb, 16)).astype(np.int8).view(np.uint8)
    d = rng.uniform(2.0 ** -12, 2.0 ** -8, size=n_rows * nb).astype(np.float16)
    blk[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return blk.reshape(n_rows, nb * Q6K_BYTES)


def q6k_dequant(w, n_cols):
    """float64 [n_rows, n_cols]: weight = d * sc * (u - 32), u the 6-bit value
    (low 4 bits from ql, high 2 from qh), sc the int8 scale of its 16-group."""
    n_rows = w.shape[0]
    nb = n_cols // 256
    blk = w.reshape(n_rows * nb, Q6K_BYTES).astype(np.int64)
    d = w.reshape(n_rows * nb, Q6K_BYTES)[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
    sc = w.reshape(n_rows * nb, Q6K_BYTES)[:, 192:208].copy().view(np.int8).astype(np.float64)
    out = np.zeros((n_rows * nb, 256))
    for half in range(2):
        ql = blk[:, 64 * half:64 * half + 64]
        qh = blk[:, 128 + 32 * half:128 + 32 * half + 32]
        base = 128 * half
        for l in range(32):
            us = [(ql[:, l] & 0xF) | ((qh[:, l] & 3) << 4), (ql[:, l + 32] & 0xF) | ((qh[:, l] & 0xC) << 2),
                  (ql[:, l] >> 4) | (qh[:, l] & 0x30), (ql[:, l + 32] >> 4) | ((qh[:, l] & 0xC0) >> 2)]
            for k, u in enumerate(us):
                idx = base + 32 * k + l
                out[:, idx] = d * sc[:, idx // 16] * (u - 32)
    return out.reshape(n_rows, n_cols)


# -- Q4_0 / Q8_0 / Q5_K / IQ4_XS (GGML ids 2, 8, 13, 23) ------------------------
Q_BYTES_256 = {2: 144, 8: 272, 12: 144, 13: 176, 14: 210, 23: 136}  # bytes per 256 weights
IQ4NL_GRID = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                      np.int64)


def _fp16_bytes(rng, n, lo, hi):
    return rng.uniform(lo, hi, size=n).astype(np.float16).view(np.uint8).reshape(-1, 2)


def q_random(rng, qtype, n_rows, n_cols):
    """Random rows of a weight type: every quant bit random, scales fp16 in a
    range that keeps products in the usual magnitude."""
    if qtype == 12:
        return q4k_random(rng, n_rows, n_cols)
    if qtype == 14:
        return q6k_random(rng, n_rows, n_cols)
    nbytes = Q_BYTES_256[qtype] * (n_cols // 256)
    w = rng.integers(0, 256, size=(n_rows, nbytes), dtype=np.uint8)
    if qtype in (2, 8):
        bs = 18 if qtype == 2 else 34
        blk = w.reshape(-1, bs)
        blk[:, 0:2] = _fp16_bytes(rng, blk.shape[0], 2.0 ** -9, 2.0 ** -5)
    elif qtype == 13:
        blk = w.reshape(-1, 176)
        blk[:, 0:2] = _fp16_bytes(rng, blk.shape[0], 2.0 ** -10, 2.0 ** -6)
        blk[:, 2:4] = _fp16_bytes(rng, blk.shape[0], 2.0 ** -10, 2.0 ** -6)
    elif qtype == 23:
        blk = w.reshape(-1, 136)
        blk[:, 0:2] = _fp16_bytes(rng, blk.shape[0], 2.0 ** -12, 2.0 ** -8)
    return w


def q_dequant(w, qtype, n_cols):
    """float64 [n_rows, n_cols] weights from the format definitions:
    Q4_0 d*(nibble-8) (element l low nibble of qs[l], l+16 high nibble);
    Q8_0 d*q; Q5_K d*sc*(q4 + 16*qh bit) - dmin*m (chunk c of 64: low
    nibbles of qs[32c..] with qh bit 2c, high nibbles with bit 2c+1);
    IQ4_XS d*(6-bit scale - 32)*grid[nibble]."""
    if qtype == 12:
        return q4k_dequant(w, n_cols)
    if qtype == 14:
        return q6k_dequant(w, n_cols)
    n_rows = w.shape[0]
    f16 = lambda a: a.copy().view(np.float16).astype(np.float64)[:, 0]
    if qtype in (2, 8):
        bs = 18 if qtype == 2 else 34
        blk = w.reshape(-1, bs)
        d = f16(blk[:, 0:2])
        if qtype == 2:
            qs = blk[:, 2:18].astype(np.int64)
            q = np.concatenate([qs & 0xF, qs >> 4], axis=1) - 8
        else:
            q = blk[:, 2:34].copy().view(np.int8).astype(np.int64)
        return (d[:, None] * q).reshape(n_rows, n_cols)
    nb = n_cols // 256
    if qtype == 13:
        blk = w.reshape(n_rows * nb, 176)
        d, dm = f16(blk[:, 0:2]), f16(blk[:, 2:4])
        sc_bytes = blk[:, 4:16].astype(np.int64)
        qh = blk[:, 16:48].astype(np.int64)
        qs = blk[:, 48:176].astype(np.int64)
        out = np.zeros((n_rows * nb, 256))
        for j in range(8):
            sc, m = _q4k_scale_min(sc_bytes, j)
            c = j // 2
            nib = (qs[:, 32 * c:32 * c + 32] & 0xF) if j % 2 == 0 else (qs[:, 32 * c:32 * c + 32] >> 4)
            q = nib + 16 * ((qh >> j) & 1)
            out[:, 32 * j:32 * j + 32] = (d * sc)[:, None] * q - (dm * m)[:, None]
        return out.reshape(n_rows, n_cols)
    if qtype == 23:
        blk = w.reshape(n_rows * nb, 136)
        d = f16(blk[:, 0:2])
        sh = blk[:, 2:4].copy().view(np.uint16).astype(np.int64)[:, 0]
        sl = blk[:, 4:8].astype(np.int64)
        qs = blk[:, 8:136].astype(np.int64)
        out = np.zeros((n_rows * nb, 256))
        for ib in range(8):
            ls = (((sl[:, ib >> 1] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4)) - 32
            sub = qs[:, 16 * ib:16 * ib + 16]
            vals = np.concatenate([IQ4NL_GRID[sub & 0xF], IQ4NL_GRID[sub >> 4]], axis=1)
            out[:, 32 * ib:32 * ib + 32] = (d * ls)[:, None] * vals
        return out.reshape(n_rows, n_cols)
    raise ValueError(qtype)
