"""GPU parity of the engine context's KV persistence: .lfmcache v1 files
(lfm_attn_ctx_cache_save / lfm_attn_ctx_cache_load_prefix) and the checkpoint
SWA slab (lfm_attn_ctx_swa_slab_save / _restore), against the oracle
(oracle/cpu_cache.c, pinned byte-identical to the reference's writer, loader
and checkpoint in test_cache_oracle.py).

The context's caches are filled by its own forward steps, so the files carry
what the HIP prologue wrote; files must be byte-identical to the oracle's
file of the exported caches, a restored context must continue bit-identically,
and a rejected file must leave caches and states untouched."""
import os

import numpy as np
import pytest

from oracle.bindings import CacheModel

pytestmark = pytest.mark.gpu

NQ, NKV, HD = 16, 4, 64


def make_ctx(la, kinds, max_seq, win=0, cap=0):
    """Context holding the attention layers of a model with layer kinds
    `kinds` (0 ShortConv, 1 full, 2 SWA); returns (ctx, oracle model, ctx_layer)."""
    attn = [k for k in kinds if k]
    lfm3 = any(k == 2 for k in kinds)
    kw = {}
    if lfm3:
        kw = dict(lfm3=True, sliding_window=win, swa_cap=cap, layer_is_swa=[k == 2 for k in attn],
                  rope_base_swa=1e4, rope_dim=HD)
    ctx = la.EngineContext(len(attn), NQ, NKV, HD, max_seq, 1e-5, rope_base=1e6, **kw)
    model = CacheModel(kinds, [NKV if k else 0 for k in kinds], HD, NQ * HD, NQ, l_cache=3,
                       sliding_window=win, is_lfm3=lfm3)
    ctx_layer, i = [], 0
    for k in kinds:
        ctx_layer.append(i if k else -1)
        i += 1 if k else 0
    return ctx, model, ctx_layer


def run(ctx, n_attn, pos_0, B, rng):
    outs = []
    for layer in range(n_attn):
        q = rng.standard_normal((B, NQ, HD), dtype=np.float32)
        k = rng.standard_normal((B, NKV, HD), dtype=np.float32)
        v = rng.standard_normal((B, NKV, HD), dtype=np.float32)
        outs.append(ctx.forward(layer, pos_0, q, k, v))
    return outs


def fill(ctx, n_attn, n_tokens, rng):
    pos = 0
    while pos < n_tokens:
        B = min(int(rng.choice([1, 3, 8])), n_tokens - pos)
        run(ctx, n_attn, pos, B, rng)
        pos += B


def host_caches(ctx, model, ctx_layer):
    """Whole device caches of every model layer (None for ShortConv)."""
    k, v = [], []
    for l, cl in enumerate(ctx_layer):
        if cl < 0:
            k.append(None)
            v.append(None)
            continue
        slots = ctx.slots(cl)
        kh, vh = ctx.kv_export(cl, 0, slots)
        k.append(kh.reshape(-1))
        v.append(vh.reshape(-1))
    return k, v


def conv_states(rng, model):
    return [rng.standard_normal(2 * model.n_embd).astype(np.float32) if kind == 0 else None
            for kind in model.layer_kind]


@pytest.mark.parametrize("kinds,n_tokens,win,cap", [
    ([0, 1, 0, 1, 0], 37, 0, 0),             # LFM2 hybrid: ShortConv + full attention
    ([0, 2, 1, 2, 0], 45, 16, 24),           # LFM3: the SWA ring wrapped
    ([0, 2, 1, 2, 0], 11, 16, 24),           # LFM3: fewer tokens than the window
])
def test_save_matches_oracle_and_restores(gpu, orc, tmp_path, kinds, n_tokens, win, cap):
    la = gpu
    rng = np.random.default_rng(n_tokens)
    max_seq = 128
    a, model, ctx_layer = make_ctx(la, kinds, max_seq, win, cap)
    n_attn = sum(1 for k in kinds if k)
    fill(a, n_attn, n_tokens, rng)
    tokens = rng.integers(0, 65536, 80, dtype=np.uint32)
    conv = conv_states(rng, model)
    heads = [1 if kind == 0 else 0 for kind in kinds]
    fp = orc.model_fingerprint(model)
    pm = la.CacheModel(fp, ctx_layer, model.n_embd, model.n_head_q, model.l_cache)
    path, want = str(tmp_path / "gpu.lfmcache"), str(tmp_path / "orc.lfmcache")
    a.cache_save(path, pm, tokens[:n_tokens], conv, heads)
    k, v = host_caches(a, model, ctx_layer)
    assert orc.prompt_cache_save(want, model, tokens[:n_tokens], conv, k, v, conv_heads=heads,
                                 swa_cap=cap, fingerprint=fp)
    assert open(path, "rb").read() == open(want, "rb").read()
    assert not [f for f in os.listdir(tmp_path) if ".tmp." in f]

    # restore into a fresh context: same states, same rows, same continuation
    b, _, _ = make_ctx(la, kinds, max_seq, win, cap)
    conv2 = [None if c is None else np.zeros_like(c) for c in conv]
    matched, got_heads = b.cache_load_prefix(path, pm, tokens, conv2)
    assert matched == n_tokens
    for l, c in enumerate(conv):
        if c is not None:
            lin = c.reshape(2, -1)[[(heads[l] + s) % 2 for s in range(2)]].reshape(-1)
            assert np.array_equal(conv2[l], lin) and got_heads[l] == 0
    kb, vb = host_caches(b, model, ctx_layer)
    ko, vo = [None if x is None else np.zeros_like(x) for x in k], [None if x is None else np.zeros_like(x) for x in v]
    assert orc.prompt_cache_load(want, model, tokens, max_seq, [None] * len(kinds), ko, vo, swa_cap=cap,
                                 fingerprint=fp)[0] == n_tokens
    for x, y in zip(kb + vb, ko + vo):
        assert (x is None and y is None) or np.array_equal(x, y)
    s1, s2 = np.random.default_rng(5), np.random.default_rng(5)
    for pos in (n_tokens, n_tokens + 1):
        for x, y in zip(run(a, n_attn, pos, 1, s1), run(b, n_attn, pos, 1, s2)):
            assert np.array_equal(x, y)
    a.close()
    b.close()


@pytest.mark.parametrize("case", ["mismatch", "short_prompt", "fingerprint", "checksum", "kv_byte",
                                  "truncate", "past_max_seq", "missing"])
def test_rejected_file_leaves_context_untouched(gpu, orc, tmp_path, case):
    la = gpu
    rng = np.random.default_rng(7)
    kinds = [0, 2, 1, 2, 0]
    a, model, ctx_layer = make_ctx(la, kinds, 64, 16, 24)
    fill(a, 3, 30, rng)
    tokens = rng.integers(0, 65536, 40, dtype=np.uint32)
    fp = orc.model_fingerprint(model)
    pm = la.CacheModel(fp, ctx_layer, model.n_embd, model.n_head_q, model.l_cache)
    path = str(tmp_path / "c.lfmcache")
    a.cache_save(path, pm, tokens[:30], conv_states(rng, model))
    b, _, _ = make_ctx(la, kinds, 64 if case != "past_max_seq" else 29, 16, 24)
    fill(b, 3, 20, rng)
    before = host_caches(b, model, ctx_layer)
    conv = conv_states(rng, model)
    conv_before = [None if c is None else c.copy() for c in conv]
    prompt, lm = tokens, pm
    data = bytearray(open(path, "rb").read())
    if case == "mismatch":
        prompt = tokens.copy()
        prompt[17] ^= 1
    elif case == "short_prompt":
        prompt = tokens[:29]
    elif case == "fingerprint":
        lm = la.CacheModel(fp ^ 1, ctx_layer, model.n_embd, model.n_head_q, model.l_cache)
    elif case == "checksum":
        data[-3] ^= 0x10
    elif case == "kv_byte":
        data[64 + 30 * 4 + 2 * 1024 * 4 + 10] ^= 0x01   # a K row of the first SWA layer
    elif case == "truncate":
        data = data[:-9]
    elif case == "missing":
        path = str(tmp_path / "absent.lfmcache")
    if case in ("checksum", "kv_byte", "truncate"):
        open(path, "wb").write(bytes(data))
    matched, _ = b.cache_load_prefix(path, lm, prompt, conv)
    assert matched == 0
    after = host_caches(b, model, ctx_layer)
    for x, y in zip(before[0] + before[1], after[0] + after[1]):
        assert (x is None and y is None) or np.array_equal(x, y)
    for x, y in zip(conv, conv_before):
        assert (x is None and y is None) or np.array_equal(x, y)
    a.close()
    b.close()


def test_save_errors(gpu, orc, tmp_path):
    la = gpu
    kinds = [0, 1]
    a, model, ctx_layer = make_ctx(la, kinds, 32)
    fill(a, 1, 10, np.random.default_rng(1))
    pm = la.CacheModel(orc.model_fingerprint(model), ctx_layer, model.n_embd, model.n_head_q, 3)
    conv = conv_states(np.random.default_rng(2), model)
    with pytest.raises(la.LfmAttnError) as e:
        a.cache_save(str(tmp_path / "x"), pm, np.arange(33, dtype=np.uint32), conv)
    assert e.value.status == -2                        # past max_seq
    with pytest.raises(la.LfmAttnError) as e:
        a.cache_save(str(tmp_path / "no_dir" / "x"), pm, np.arange(10, dtype=np.uint32), conv)
    assert e.value.status == -6                        # cannot write
    with pytest.raises(la.LfmAttnError) as e:
        a.cache_save(str(tmp_path / "x"), pm, np.arange(10, dtype=np.uint32), None)
    assert e.value.status == -1                        # ShortConv layer without a state
    bad = la.CacheModel(pm.fingerprint, [-1, 1], model.n_embd, model.n_head_q, 3)
    with pytest.raises(la.LfmAttnError) as e:
        a.cache_save(str(tmp_path / "x"), bad, np.arange(10, dtype=np.uint32), conv)
    assert e.value.status == -1                        # no such context layer
    assert not os.listdir(tmp_path)
    a.close()


def test_checkpoint_slab_and_rollback(gpu, orc):
    """Slab == the oracle's (reference layout) of the exported rings; after
    overwriting the ring, restoring the slab (host or device) and replaying
    the same steps gives bit-identical outputs."""
    la = gpu
    rng = np.random.default_rng(3)
    kinds = [0, 2, 1, 2]
    win, cap = 16, 24
    a, model, ctx_layer = make_ctx(la, kinds, 128, win, cap)
    fill(a, 3, 40, rng)
    assert a.swa_slab_bytes() == 2 * 2 * cap * NKV * HD * 2
    slab = a.swa_slab_save()
    k, v = host_caches(a, model, ctx_layer)
    assert np.array_equal(slab, orc.checkpoint_swa_slab(model, cap, k, v))
    dslab = la.DeviceArray.zeros(slab.size, np.uint16)
    a.swa_slab_save(dslab)
    assert np.array_equal(dslab.numpy(), slab)

    steps = [(40, 3), (43, 8), (51, 1), (52, 8)]   # 20 positions: the ring turns over
    first = []
    for pos, B in steps:
        first += run(a, 3, pos, B, np.random.default_rng(pos))
    for src in (slab, dslab):
        a.swa_slab_restore(src)
        again = []
        for pos, B in steps:
            again += run(a, 3, pos, B, np.random.default_rng(pos))
        for x, y in zip(first, again):
            assert np.array_equal(x, y)
    k2, v2 = host_caches(a, model, ctx_layer)
    a.swa_slab_restore(slab)
    k3, v3 = host_caches(a, model, ctx_layer)
    for l in (1, 3):
        assert np.array_equal(k3[l], k[l]) and np.array_equal(v3[l], v[l])
    assert np.array_equal(k3[2], k2[2])  # full layers are not part of the slab
    a.close()
