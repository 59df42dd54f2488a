"""Shared input builders and the parity bar for the tests."""
from __future__ import annotations

import numpy as np

# fp32 outputs within max-abs 2e-3 and relative L2 1e-3
# of the CPU reference on the same inputs.
MAX_ABS = 2e-3
REL_L2 = 1e-3


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
