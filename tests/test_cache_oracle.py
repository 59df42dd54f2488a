"""KV persistence formats beside the attention path: pins of the oracle's
.lfmcache v1 writer/loader and checkpoint SWA slab (oracle/cpu_cache.c).

- FNV-1a 64 against its published test vectors.
- The model fingerprint against lfm2_compute_model_fingerprint
  (tools/lfm2_sys_cache.c:394-422) compiled from the reference.
- Files byte-identical to lfm2_prompt_cache_save_ex
  (tools/lfm2_sys_cache.c:504-627); each loader accepts the other's files and
  both make the same accept/reject decision
  (lfm2_prompt_cache_try_load_prefix_ex, :650-797).
- The reference's own cases: tests/test_sys_cache.c:200-410 (round trip,
  prefix rule, tampered byte at offset 75) and the LFM3 SWA case of
  tests/test_lfm3.c:440-510 (15 tokens > window 8, ring heads).
- The checkpoint slab against lfm2_checkpoint_save_ex / restore_ex
  (tools/lfm2_moe_checkpoint.c:399-560)."""
import os
import struct

import numpy as np
import pytest

from oracle.bindings import CacheModel

MAGIC = 0x4350324D464C3130


def lfm2_unit_model():
    """tests/test_sys_cache.c:203-215: layers 0, 1, 3 ShortConv, layer 2 GQA."""
    return CacheModel([0, 0, 1, 0], [0, 0, 2, 0], head_dim=64, n_embd=256, n_head_q=4, l_cache=3)


def unit_buffers(m, n_tokens):
    """The fill patterns of tests/test_sys_cache.c:225-241."""
    conv, k, v = [], [], []
    for l in range(m.n_layers):
        if m.layer_kind[l] == 0:
            conv.append((np.arange(2 * m.n_embd, dtype=np.float32) + np.float32(l * 500)) * np.float32(1.5))
            k.append(None)
            v.append(None)
        else:
            kv = int(m.n_head_kv[l]) * m.head_dim
            i = np.arange(n_tokens * kv, dtype=np.int64)
            conv.append(None)
            k.append(((l * 100 + i) & 0x7FFF).astype(np.uint16))
            v.append(((l * 200 + i) & 0x7FFF).astype(np.uint16))
    return conv, k, v


def lfm3_model(win=8):
    return CacheModel([0, 2, 1, 2, 0], [0, 2, 4, 2, 0], head_dim=64, n_embd=128, n_head_q=8,
                      l_cache=4, sliding_window=win, is_lfm3=True)


def random_buffers(rng, m, rows_full, cap):
    conv, k, v = [], [], []
    for l in range(m.n_layers):
        kind = int(m.layer_kind[l])
        if kind == 0:
            conv.append(rng.standard_normal(m.hist_len * m.n_embd).astype(np.float32))
            k.append(None)
            v.append(None)
            continue
        rows = rows_full if kind == 1 else cap
        kv = int(m.n_head_kv[l]) * m.head_dim
        conv.append(None)
        k.append(rng.integers(0, 1 << 16, rows * kv, dtype=np.uint16))
        v.append(rng.integers(0, 1 << 16, rows * kv, dtype=np.uint16))
    return conv, k, v


def zeros_like(bufs):
    return [None if b is None else np.zeros_like(b) for b in bufs]


def test_fnv1a_published_vectors(orc):
    assert orc.fnv1a(b"") == 0xCBF29CE484222325
    assert orc.fnv1a(b"a") == 0xAF63DC4C8601EC8C
    assert orc.fnv1a(b"foobar") == 0x85944171F73967E8


@pytest.mark.parametrize("model", [lfm2_unit_model(), lfm3_model(8), lfm3_model(256),
                                   CacheModel([0, 1] * 8, [0, 8] * 8, 64, 2048, 32, 3)])
def test_fingerprint_matches_reference(orc, ref, model):
    assert orc.model_fingerprint(model) == ref.model_fingerprint(model)


def test_fingerprint_separates_models(orc):
    a = orc.model_fingerprint(lfm2_unit_model())
    other = CacheModel([0, 0, 1, 0], [0, 0, 2, 0], 64, 128, 4, 3)   # n_embd differs
    assert a != orc.model_fingerprint(other)
    # LFM3 hashes the window and the SWA layer map too
    assert orc.model_fingerprint(lfm3_model(8)) != orc.model_fingerprint(lfm3_model(16))


def test_unit_round_trip_and_bytes(orc, ref, tmp_path):
    """tests/test_sys_cache.c:200-289: 32 cached tokens, prompt of 48."""
    m = lfm2_unit_model()
    tokens = np.array([1000 + 3 * i for i in range(48)], np.uint32)
    conv, k, v = unit_buffers(m, 32)
    po, pr = str(tmp_path / "o.lfmcache"), str(tmp_path / "r.lfmcache")
    assert orc.prompt_cache_save(po, m, tokens[:32], conv, k, v)
    assert ref.prompt_cache_save(pr, m, tokens[:32], conv, k, v)
    data = open(po, "rb").read()
    assert data == open(pr, "rb").read()
    # header fields and size
    magic, ver, n, fp, nl, ne, nhq, lc, payload = struct.unpack_from("<QIIQIIIIQ", data)
    assert (magic, ver, n, nl, ne, nhq, lc) == (MAGIC, 1, 32, 4, 256, 4, 3)
    assert fp == orc.model_fingerprint(m)
    assert payload == 32 * 4 + 3 * 2 * 256 * 4 + 2 * 32 * 128 * 2
    assert len(data) == 64 + payload + 8
    assert struct.unpack_from("<Q", data, len(data) - 8)[0] == orc.fnv1a(data[64:-8])
    assert not [f for f in os.listdir(tmp_path) if ".tmp." in f]
    for path in (po, pr):
        for lib in (orc, ref):
            c2, k2, v2 = zeros_like(conv), zeros_like(k), zeros_like(v)
            matched, heads = lib.prompt_cache_load(path, m, tokens, 512, c2, k2, v2)
            assert matched == 32
            for a, b in zip(c2 + k2 + v2, conv + k + v):
                assert (a is None and b is None) or np.array_equal(a, b)
            assert all(heads[l] == 0 for l in (0, 1, 3))


def prefix_rule_model():
    """tests/test_sys_cache.c:294-303"""
    return CacheModel([0, 1], [0, 1], 64, 64, 1, 3)


@pytest.mark.parametrize("case", ["mismatch", "short_prompt", "fingerprint", "max_seq"])
def test_prefix_rule_rejections(orc, ref, tmp_path, case):
    """tests/test_sys_cache.c:291-353 plus the max_seq bound of :701."""
    m = prefix_rule_model()
    cached = np.arange(1, 17, dtype=np.uint32)
    conv = [np.zeros(2 * 64, np.float32), None]
    k = [None, np.zeros(16 * 64, np.uint16)]
    v = [None, np.zeros(16 * 64, np.uint16)]
    path = str(tmp_path / "p.lfmcache")
    assert orc.prompt_cache_save(path, m, cached, conv, k, v)
    prompt, lm, max_seq = cached, m, 512
    if case == "mismatch":
        prompt = np.array([999 if i == 5 else i + 1 for i in range(20)], np.uint32)
    elif case == "short_prompt":
        prompt = cached[:10]
    elif case == "fingerprint":
        lm = CacheModel([0, 1], [0, 1], 64, 128, 1, 3)
    else:
        max_seq = 15
    for lib in (orc, ref):
        matched, _ = lib.prompt_cache_load(path, lm, prompt, max_seq, conv, k, v)
        assert matched == 0
    # the exact prefix with a longer prompt is accepted
    assert orc.prompt_cache_load(path, m, np.arange(1, 40, dtype=np.uint32), 512, conv, k, v)[0] == 16


@pytest.mark.parametrize("offset", [75, 64 + 32 + 100, -9, -1, "truncate"])
def test_tampered_or_truncated_rejected(orc, ref, tmp_path, offset):
    """tests/test_sys_cache.c:356-405 (byte 75, in the token ids), plus a
    ShortConv byte, the last payload byte, the checksum and a cut file."""
    m = prefix_rule_model()
    tokens = np.arange(1, 9, dtype=np.uint32)
    conv = [np.linspace(-1, 1, 128).astype(np.float32), None]
    k = [None, np.arange(8 * 64, dtype=np.uint16)]
    v = [None, np.arange(8 * 64, dtype=np.uint16)[::-1].copy()]
    path = str(tmp_path / "c.lfmcache")
    assert orc.prompt_cache_save(path, m, tokens, conv, k, v)
    data = bytearray(open(path, "rb").read())
    if offset == "truncate":
        data = data[:-20]
    else:
        data[offset] ^= 0xFF
    open(path, "wb").write(bytes(data))
    for lib in (orc, ref):
        assert lib.prompt_cache_load(path, m, tokens, 512, zeros_like(conv), zeros_like(k),
                                     zeros_like(v))[0] == 0


@pytest.mark.parametrize("n_tokens,heads", [(15, [1, 0, 0, 0, 2]), (5, [0, 0, 0, 0, 0]),
                                            (8, [2, 0, 0, 0, 1]), (40, [1, 0, 0, 0, 1])])
def test_lfm3_swa_ring_bytes_and_load(orc, ref, tmp_path, n_tokens, heads):
    """LFM3 layout (tests/test_lfm3.c:440-510): SWA layers keep the last
    min(n, window) positions from ring slot t % (window + 8); the ShortConv
    ring is linearized from its head; the loader returns heads 0."""
    win, cap = 8, 16
    m = lfm3_model(win)
    rng = np.random.default_rng(n_tokens)
    conv, k, v = random_buffers(rng, m, 64, cap)
    tokens = rng.integers(0, 65536, 64, dtype=np.uint32)
    po, pr = str(tmp_path / "o.lfmcache"), str(tmp_path / "r.lfmcache")
    assert orc.prompt_cache_save(po, m, tokens[:n_tokens], conv, k, v, conv_heads=heads, swa_cap=cap)
    assert ref.prompt_cache_save(pr, m, tokens[:n_tokens], conv, k, v, conv_heads=heads, swa_cap=cap)
    assert open(po, "rb").read() == open(pr, "rb").read()
    for lib in (orc, ref):
        c2, k2, v2 = zeros_like(conv), zeros_like(k), zeros_like(v)
        matched, got_heads = lib.prompt_cache_load(po, m, tokens, 64, c2, k2, v2, swa_cap=cap)
        assert matched == n_tokens
        hist = m.hist_len
        for l in (0, 4):
            ring = conv[l].reshape(hist, -1)
            lin = ring[[(heads[l] + s) % hist for s in range(hist)]]
            assert np.array_equal(c2[l].reshape(hist, -1), lin) and got_heads[l] == 0
        kv = 2 * 64
        for l in (1, 3):
            slots = [t % cap for t in range(max(0, n_tokens - win), n_tokens)]
            for src, dst in ((k[l], k2[l]), (v[l], v2[l])):
                s2, d2 = src.reshape(cap, kv), dst.reshape(cap, kv)
                assert np.array_equal(d2[slots], s2[slots])
                others = [s for s in range(cap) if s not in slots]
                assert not d2[others].any()
        assert np.array_equal(k2[2].reshape(64, -1)[:n_tokens], k[2].reshape(64, -1)[:n_tokens])


def test_checkpoint_swa_slab_matches_reference(orc, ref):
    """The slab is every SWA layer's whole K ring then V ring in layer order,
    with rings of window + 8 slots."""
    m = lfm3_model(8)
    cap = 16
    rng = np.random.default_rng(21)
    _, k, v = random_buffers(rng, m, 32, cap)
    slab = orc.checkpoint_swa_slab(m, cap, k, v)
    assert np.array_equal(slab, ref.checkpoint_swa_save(m, k, v))
    ring = cap * 2 * 64
    assert slab.size == 4 * ring
    assert np.array_equal(slab[:ring], k[1]) and np.array_equal(slab[ring:2 * ring], v[1])
    assert np.array_equal(slab[2 * ring:3 * ring], k[3])
    k2, v2 = zeros_like(k), zeros_like(v)
    k3, v3 = zeros_like(k), zeros_like(v)
    orc.checkpoint_swa_slab(m, cap, k2, v2, slab=slab)
    assert ref.checkpoint_swa_restore(m, slab, k3, v3)
    for l in (1, 3):
        assert np.array_equal(k2[l], k[l]) and np.array_equal(v2[l], v[l])
        assert np.array_equal(k3[l], k[l]) and np.array_equal(v3[l], v[l])
    assert not k2[2].any() and not k3[2].any()  # full layers are not in the slab


def _fnv_chunked(data, h0, chunk=64, fan=4):
    """numpy emulation of the device decomposition of FNV-1a 64: per-chunk
    256-state maps of the low byte, composed in groups into prefix tables,
    then each chunk's polynomial from its start state, weighted by
    P^(bytes after it)."""
    P, M = 0x100000001B3, (1 << 64) - 1
    states = np.arange(256, dtype=np.int64)
    n = (len(data) + chunk - 1) // chunk
    maps = []
    for c in range(n):
        s = states.copy()
        for b in data[c * chunk:(c + 1) * chunk]:
            s = ((s ^ int(b)) * 179) & 255
        maps.append(s)
    levels, cur = [], maps
    while len(cur) > 1:
        pre, up = [], []
        for g in range(0, len(cur), fan):
            s = states.copy()
            for m in cur[g:g + fan]:
                pre.append(s.copy())
                s = m[s]
            up.append(s)
        levels.append(pre)
        cur = up
    acc = 0
    for i in range(n):
        s = h0 & 255
        for l in range(len(levels) - 1, -1, -1):
            s = int(levels[l][i // fan ** l][s])
        a = 0
        seg = data[i * chunk:(i + 1) * chunk]
        for b in seg:
            x = s ^ int(b)
            a = ((a + (x - s)) * P) & M
            s = (x * 179) & 255
        acc = (acc + a * pow(P, len(data) - i * chunk - len(seg), 1 << 64)) & M
    return (h0 * pow(P, len(data), 1 << 64) + acc) & M


def test_low_byte_map_bit7_symmetry():
    """map(s ^ 128) = map(s) ^ 128 for any byte run, so the device runs only
    states 0..127 (128 * 179 = 128 mod 256)."""
    rng = np.random.default_rng(4)
    states = np.arange(256, dtype=np.int64)
    for n in (1, 7, 300):
        s = states.copy()
        for b in rng.integers(0, 256, n):
            s = ((s ^ int(b)) * 179) & 255
        assert np.array_equal(s[128:], s[:128] ^ 128)
        assert sorted(s.tolist()) == list(range(256))  # a permutation


@pytest.mark.parametrize("n", [1, 63, 64, 65, 64 * 4 * 4 + 7, 1500])
def test_parallel_fnv_decomposition(orc, n):
    """The identity the device hash relies on, checked against the sequential
    FNV-1a on small buffers and uneven chunk counts (several levels)."""
    rng = np.random.default_rng(n)
    data = rng.integers(0, 256, n, dtype=np.uint8)
    for h0 in (14695981039346656037, 0x1234567890ABCDEF):
        assert _fnv_chunked(data, h0) == orc.fnv1a(data, h0)
